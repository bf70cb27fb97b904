"""The C-ABI library: it loads, exports every symbol include/gpu.h declares,
and its host-only paths behave as specified — CPU only, no device calls."""
import ctypes as C
import os
import re

import numpy as np

import fomoe_amd
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(ROOT, "include", "gpu.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(gpu_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(fomoe_amd.LIB_PATH)
    names = declared_symbols()
    assert "gpu_expert_ffn" in names and "gpu_moe_layer" in names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers each of them with a signature
    assert sorted(fomoe_amd.SIGNATURES) == names


def test_library_is_gfx950_only():
    blob = open(fomoe_amd.LIB_PATH, "rb").read()
    assert b"gfx950" in blob
    for other in (b"gfx1200", b"gfx942", b"gfx90a", b"sm_80"):
        assert other not in blob


def test_expert_ffn_null_ctx_and_limits_fall_back():
    """gpu_expert_ffn returns -1 ("use the CPU") for a NULL context before any
    device work, as reference gpu_kernels.hip:8393."""
    lib = fomoe_amd.load_library()
    h = np.zeros(4096, np.float32)
    out = np.zeros(4096, np.float32)
    rc = lib.gpu_expert_ffn(None, h.ctypes.data, None, None, 10, 4096, 1024, 0, 0, 0,
                            12, 12, 14, out.ctypes.data)
    assert rc == -1
    assert lib.gpu_sync(None) == -1
    assert lib.gpu_matvec_q(None, 12, None, None, None, 1, 256) == -1
    assert lib.gpu_alloc(None, 16) is None


def test_zipf_bias_matches_oracle():
    lib = fomoe_amd.load_library()
    for seed, st, n in ((4, 6, 512), (9, 123, 64)):
        got = np.empty(n, np.float32)
        lib.gpu_synth_zipf_bias(seed, st, n, 1.1, got.ctypes.data)
        assert np.array_equal(got, O.zipf_bias(seed, st, n, 1.1))


def test_struct_layouts_match_header():
    """gpu_moe_layer_t field order/offsets equal the oracle's descriptor."""
    a, b = fomoe_amd.MoeLayer, O.MoeDesc
    assert [f[0] for f in a._fields_] == [f[0] for f in b._fields_]
    assert C.sizeof(a) == C.sizeof(b)
