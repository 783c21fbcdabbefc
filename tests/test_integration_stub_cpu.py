"""The reference-side ctypes binding printed in INTEGRATION.md section 3 works against the built
library (no GPU: every call carries a batch of zero sequences, which the library accepts after its
argument checks without touching device memory).

The code block is executed as written, with only its ``.so`` path replaced by the built one, so
that an ABI change (a field added to a struct, a new version number) that is not copied into the
document turns this test red: the block's own version assert, its struct layouts against
``lastkv_amd._lib`` (which mirrors ``include/lastkv_amd.h`` field for field), the fields its
functions set, and one call of each function through the library.
"""

from __future__ import annotations

import ast
import ctypes
import pathlib
import re

import torch

from lastkv_amd import _lib

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _stub_source() -> str:
    text = (ROOT / "INTEGRATION.md").read_text()
    section = text[text.index("## 3. Binding the C ABI directly"):text.index("## 4.")]
    blocks = re.findall(r"```python\n(.*?)```", section, flags=re.S)
    assert len(blocks) == 1, "section 3 must hold exactly one python block (the stub)"
    assert '"/opt/lastkv/liblastkv_amd.so"' in blocks[0]
    return blocks[0]


def _load_stub() -> dict:
    src = _stub_source().replace('"/opt/lastkv/liblastkv_amd.so"', repr(str(_lib.LIB_PATH)))
    _lib.load()  # builds nothing; raises if the library is missing
    ns: dict = {}
    exec(compile(src, "INTEGRATION.md#3", "exec"), ns)  # runs the block's version assert
    return ns


def test_header_and_python_mirror_agree_on_the_abi_version():
    header = (ROOT / "include" / "lastkv_amd.h").read_text()
    version = int(re.search(r"#define LKV_ABI_VERSION (\d+)", header).group(1))
    assert version == _lib.ABI_VERSION == _lib.load().lkv_abi_version()
    assert f"assert _lib.lkv_abi_version() == {version}" in _stub_source()


def test_stub_struct_layouts_equal_the_header():
    ns = _load_stub()
    for stub_name, mirror in (("lkv_decode_args", _lib.DecodeArgs), ("lkv_prefill_args", _lib.PrefillArgs)):
        stub = ns[stub_name]
        assert ctypes.sizeof(stub) == ctypes.sizeof(mirror), stub_name
        assert [(n, t) for n, t in stub._fields_] == [(n, t) for n, t in mirror._fields_], stub_name


def _assigned_fields(fn: ast.FunctionDef) -> tuple[str | None, set[str]]:
    """(struct class the function instantiates as ``a``, the ``a.<field>`` names it assigns,
    including ``setattr(a, prefix + "_suffix", ...)`` over literal prefixes)."""

    struct, names = None, set()
    prefixes: list[str] = []
    for node in ast.walk(fn):
        if isinstance(node, ast.Assign) and len(node.targets) == 1 and isinstance(node.targets[0], ast.Name):
            if node.targets[0].id == "a" and isinstance(node.value, ast.Call) and isinstance(node.value.func, ast.Name):
                struct = node.value.func.id
        if isinstance(node, (ast.Assign, ast.AugAssign)):
            targets = node.targets if isinstance(node, ast.Assign) else [node.target]
            for t in targets:
                for e in (t.elts if isinstance(t, ast.Tuple) else [t]):
                    if isinstance(e, ast.Attribute) and isinstance(e.value, ast.Name) and e.value.id == "a":
                        names.add(e.attr)
        if isinstance(node, ast.For) and isinstance(node.iter, ast.Tuple):
            for elt in node.iter.elts:
                if isinstance(elt, ast.Tuple) and elt.elts and isinstance(elt.elts[0], ast.Constant):
                    prefixes.append(elt.elts[0].value)
        if (isinstance(node, ast.Call) and isinstance(node.func, ast.Name) and node.func.id == "setattr"
                and isinstance(node.args[1], ast.BinOp) and isinstance(node.args[1].right, ast.Constant)):
            names.update(p + node.args[1].right.value for p in prefixes)
    return struct, names


def test_stub_functions_set_only_declared_fields():
    ns = _load_stub()
    tree = ast.parse(_stub_source())
    checked = 0
    for fn in (n for n in tree.body if isinstance(n, ast.FunctionDef)):
        struct, names = _assigned_fields(fn)
        if struct is None:
            continue
        fields = {n for n, _ in ns[struct]._fields_}
        assert names, fn.name
        assert names <= fields, f"{fn.name} sets undeclared fields {sorted(names - fields)}"
        assert "struct_size" in names, fn.name
        checked += 1
    assert checked == 2


class _Rows:
    """Zero query rows over real storage: torch reports a null data pointer for an empty tensor,
    which the library rejects before it looks at the batch size."""

    def __init__(self, heads: int):
        self._buf = torch.zeros(heads * 128, dtype=torch.bfloat16)
        self.shape = (0, heads, 128)

    def data_ptr(self) -> int:
        return self._buf.data_ptr()

    def stride(self, dim: int) -> int:
        return (self.shape[1] * 128, 128, 1)[dim]


def test_stub_calls_with_no_sequences_return_ok():
    ns = _load_stub()
    bf = dict(dtype=torch.bfloat16)
    i32 = dict(dtype=torch.int32)
    q, out = _Rows(8), _Rows(8)
    tiled = lambda: torch.zeros((1, 2, 1, 4096), **bf)
    ns["decode"](q, tiled(), tiled(), 0, torch.ones(2), tiled(), tiled(), 0, 0, out, None, out_scale=torch.ones(2))
    pool_k, pool_v = torch.zeros((2, 1, 4096), **bf), torch.zeros((2, 1, 4096), **bf)
    table = torch.zeros((1, 1), **i32)
    lens = torch.zeros(1, **i32)
    ns["prefill_varlen"](q, torch.zeros(1, **i32), 1, pool_k, pool_v, table, lens, table, 1, lens, lens, out,
                         torch.zeros(64, dtype=torch.uint8), None, vscale_f32=torch.ones(2), out_scale=torch.ones(2))
