"""CPU checks of the drop-in boundary: libssla_amd.so loads, exports every
symbol include/ssla_amd.h declares, and rejects bad arguments before any
device work (no GPU needed)."""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "ssla_amd.h").read_text()
    # function declarations start a line: "<type> [*]ssla_name("
    return sorted(set(re.findall(r"^(?:const\s+)?[a-z_0-9]+\s*\*?\s*(ssla_[a-z0-9_]+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from ssla_amd import _lib
    lib = _lib.load()
    names = _declared()
    assert "ssla_gla_chunk_fwd" in names and len(names) >= 10
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/ssla_amd.h but not exported"
    # the ctypes table covers the header exactly
    assert set(_lib.SIGNATURES) == set(names)


def test_version():
    from ssla_amd import _lib
    assert _lib.load().ssla_version() >= 100


def test_argument_errors_without_device_work():
    from ssla_amd import _lib
    lib = _lib.load()
    # negative sizes -> SSLA_ERR_ARG
    st = lib.ssla_gla_chunk_fwd(None, None, None, None, 0, None, -1, 0, 1, 64, 64, 1.0, None, None,
                                None, _lib.SSLA_BF16, None, 0, None)
    assert st == _lib.SSLA_ERR_ARG
    assert b"bad sizes" in lib.ssla_last_error()
    # K != 64 on the chunk kernel -> SSLA_ERR_UNSUPPORTED
    st = lib.ssla_gla_chunk_fwd(None, None, None, None, 0, None, 1, 0, 1, 32, 64, 1.0, None, None,
                                None, _lib.SSLA_BF16, None, 0, None)
    assert st == _lib.SSLA_ERR_UNSUPPORTED
    # K > 256 on the recurrent kernel
    st = lib.ssla_gla_recurrent_fwd(None, None, None, None, 0, None, 1, 0, 1, 300, 64, 1.0, None, None,
                                    None, None, 0, None, _lib.SSLA_F32, None, 0, None)
    assert st == _lib.SSLA_ERR_UNSUPPORTED
    # unsupported sparse-step shape
    st = lib.ssla_sparse_gla_step(None, 1, None, None, None, None, None, 1, 1, 48, 48, 1.0, None, None, None)
    assert st == _lib.SSLA_ERR_ARG  # null pointers are rejected first
    # scatter: non-positive C, n_out beyond 2^30, and a missing workspace
    st = lib.ssla_scatter_max(None, None, 10, 0, 4, 0, None, None, None, 0, None)
    assert st == _lib.SSLA_ERR_ARG
    st = lib.ssla_scatter_max(None, None, 10, 4, 1 << 30, 0, None, None, None, 0, None)
    assert st == _lib.SSLA_ERR_ARG
    st = lib.ssla_scatter_max(None, None, 10, 3, 4, 0, None, None, None, 0, None)
    assert st == _lib.SSLA_ERR_WORKSPACE


def test_workspace_size_monotone():
    from ssla_amd import _lib
    lib = _lib.load()
    a = lib.ssla_scatter_workspace_size(1000, 64, 100)
    b = lib.ssla_scatter_workspace_size(2000, 64, 100)
    c = lib.ssla_scatter_workspace_size(2000, 64, 200)
    assert 0 < a < b < c
    assert lib.ssla_scatter_workspace_size(-1, 64, 10) == 0


def test_chunk_forward_workspace_layout():
    """The chunk forward's workspace holds, per (sequence, head, segment), a
    K x V state as a bf16 (hi, lo) pair and K fp32 decays; C2 (8 sequences of 4096 tokens,
    8 heads) runs 8 segments per sequence, and with V = 128 (two 64-column
    groups, twice the chains) 4.  One sequence of one chunk needs no
    workspace, and unsupported shapes report 0."""
    from ssla_amd import _lib
    lib = _lib.load()
    assert lib.ssla_gla_chunk_workspace_size(8, 8 * 4096, 8, 64, 64) == 8 * 8 * 8 * (2 * 64 * 64 * 2 + 64 * 4)
    assert lib.ssla_gla_chunk_workspace_size(8, 8 * 4096, 8, 64, 128) == 8 * 8 * 4 * (2 * 64 * 128 * 2 + 64 * 4)
    assert lib.ssla_gla_chunk_workspace_size(1, 64, 8, 64, 64) == 0
    assert lib.ssla_gla_chunk_workspace_size(1, 4096, 8, 32, 64) == 0
    assert lib.ssla_gla_chunk_workspace_size(1, 4096, 8, 64, 40) == 0


def test_python_wrappers_reject_cpu_tensors():
    import torch
    from ssla_amd.gla import chunk_gla
    from ssla_amd.scan import scan
    x = torch.zeros(4, 1, 64)
    with pytest.raises(ValueError, match="device tensors"):
        chunk_gla(x, x, x, x, torch.tensor([0, 4]))
    with pytest.raises(ValueError, match="device tensors"):
        scan(torch.zeros(4, 3), torch.zeros(4, 3), torch.tensor([0, 4]))


def test_fused_mos_attention_limits():
    """The fused MosAttention kernels take at most 49 kernel positions (the
    LDS query reports 0, not applicable, beyond that even when the weights
    would fit, so the layer picks the composed forward); sizes past the
    small kernels' (hidden > 32, or weights beyond 64 KB of LDS) go to the
    matrix-core path when input and hidden are multiples of 4 up to 128."""
    from ssla_amd import _lib
    lib = _lib.load()
    assert 0 < lib.ssla_mos_attention_lds_bytes(2, 12, 49, 1, 1) <= 64 * 1024
    assert lib.ssla_mos_attention_lds_bytes(2, 12, 64, 1, 1) == 0
    for cin, hid in ((48, 48), (24, 48), (48, 96), (96, 96), (16, 32), (128, 128)):
        assert 0 < lib.ssla_mos_attention_lds_bytes(cin, hid, 9, 1, 1) <= 64 * 1024, (cin, hid)
        assert lib.ssla_mos_attention_workspace_size(1000, cin, hid, 9, 5000, 800) >= 5000 * hid * 4 * 3
    for cin, hid in ((6, 48), (48, 132), (48, 50)):
        assert lib.ssla_mos_attention_lds_bytes(cin, hid, 9, 1, 1) == 0, (cin, hid)


def test_status_read_rejects_null():
    from ssla_amd import _lib
    import ctypes
    v = ctypes.c_int(0)
    assert _lib.load().ssla_status_read(None, ctypes.byref(v), None) == _lib.SSLA_ERR_ARG


def test_struct_layouts_match_the_header(tmp_path):
    """The ctypes mirrors of the header's structs (ssla_head_level,
    ssla_grid_level) have the C compiler's field offsets and sizes."""
    import ctypes
    import shutil
    import subprocess
    from ssla_amd import _lib
    if shutil.which("gcc") is None:
        pytest.skip("no C compiler")
    structs = {"ssla_head_level": _lib.HeadLevel, "ssla_grid_level": _lib.GridLevel}
    lines = ["#include <stddef.h>", "#include <stdio.h>", f'#include "{ROOT / "include" / "ssla_amd.h"}"',
             "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'  printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-x", "c", "-I", "/opt/rocm/include", str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        name, field, val = line.split()
        got[(name, field)] = int(val)
    for cname, py in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for f, _ in py._fields_:
            assert got[(cname, f)] == getattr(py, f).offset, f"{cname}.{f}"
