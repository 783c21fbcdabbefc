"""The product path has no CPU fallback: without the built library every entry raises, and CPU
tensors are rejected before any native call (CPU tests; nothing here launches a kernel)."""

import pathlib
import subprocess
import sys
import textwrap

import pytest
import torch

from lastkv_amd import ops

REPO = pathlib.Path(__file__).resolve().parents[1]


def test_missing_library_raises_native_error():
    # a fresh process whose library path names nothing: load() and the ops built on it must raise
    code = textwrap.dedent(
        """
        import pathlib, sys
        sys.path.insert(0, sys.argv[1])
        from lastkv_amd import _lib, ops
        _lib.LIB_PATH = pathlib.Path(sys.argv[1]) / "no_such_dir" / "liblastkv_amd.so"
        for call in (_lib.load, lambda: ops.decode_workspace_bytes(1, 8, 1)):
            try:
                call()
            except _lib.LastKVNativeError as e:
                assert "is not built" in str(e), e
            else:
                raise SystemExit("no error without the library")
        print("ok")
        """
    )
    proc = subprocess.run([sys.executable, "-c", code, str(REPO)], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0 and proc.stdout.strip() == "ok", proc.stdout + proc.stderr


def test_cpu_tensors_are_rejected():
    B, Hq, Hkv, D = 1, 8, 2, 128
    q = torch.zeros(B, Hq, D, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        ops.decode_attention(q, local=ops.TiledKV.zeros(B, Hkv, 64, "cpu"), local_len=1)
