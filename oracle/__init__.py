"""CPU oracle for the LastKV shared last-layer KV attention path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg
of ``bench.py`` may import this package, and only as the checker or the timed CPU baseline; the
``lastkv_amd`` product never imports it and has no CPU fallback.

Modules:
  bf16            -- round-to-nearest-even bf16 emulation in numpy
  attention       -- fp64 softmax attention, LSE merge, LastKV region planning and the
                     reference's bf16 history composition (modeling.py:109-122)
  reference_path  -- the reference's LastKVAttention composition + SDPA restated with torch ops,
                     used as the "reference PyTorch SDPA path" and as the timed CPU baseline
  layout          -- the tiled cache layout as closed-form index maps (pack / unpack)
  model           -- the LastKV decoder restated in torch (modeling.py) plus the independent
                     eager transcription of the reference's own test (test_llm_inference.py:39-93)
  wan             -- the Wan video model's shared-history cache, previous-block blend and
                     bidirectional block attention (videogen/.../cache.py, model.py:153-272)
  vllm_path       -- the reference's vLLM serving-path rounding contract: the fused QKV kernel's
                     single-FMA rotary and RMSNorm summation order, V / s rings, the output
                     rescale and the merged per-layer op sequence (fused_qkv.py, fastpath.py:619-651)

Each function cites the reference file:line it restates; how each is pinned is stated in the
function's docstring ("pinned by: ...").
"""
