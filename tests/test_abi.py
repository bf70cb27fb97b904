"""The C-ABI library: it loads, exports every symbol include/gpu.h declares,
and its host-only paths behave as specified — CPU only, no device calls."""
import ctypes as C
import os
import re
import subprocess

import pytest

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


# Every function the reference's include/gpu.h declares (reference
# include/gpu.h:13-83); a -DQMOE_GPU build of the reference calls all of them
# (model.c:411-431, 505, 580; inference.c:427, 544; main.c:571, 882, 953-954).
REFERENCE_GPU_H = [
    "gpu_init", "gpu_free", "gpu_register_buffers", "gpu_unregister_buffers", "gpu_upload_model",
    "gpu_set_ram_cache_mb", "gpu_set_vram_cache_mb", "gpu_forward", "gpu_reset_state",
    "gpu_seed_vram_cache", "gpu_enable_expert_freq", "gpu_get_expert_freq", "gpu_get_expert_dims",
    "gpu_get_pingpong_relay_stats", "gpu_expert_ffn",
]
REF_GPU_H = "/root/reference/include/gpu.h"


def test_reference_gpu_h_names_are_exported():
    lib = C.CDLL(fomoe_amd.LIB_PATH)
    missing = [n for n in REFERENCE_GPU_H if not hasattr(lib, n)]
    assert not missing, missing
    assert set(REFERENCE_GPU_H) <= set(declared_symbols())


@pytest.mark.skipif(not os.path.exists(REF_GPU_H), reason="reference sources absent")
def test_reference_gpu_h_list_is_complete_and_signatures_agree(tmp_path):
    """The committed name list covers the reference header, and a C unit that
    includes both headers compiles: any signature that differs between the two
    declarations is a conflicting-types error."""
    src = re.sub(r"//[^\n]*", "", open(REF_GPU_H).read())
    names = set(re.findall(r"\b(gpu_[a-z0-9_]+)\s*\(", src))
    assert names == set(REFERENCE_GPU_H)
    unit = tmp_path / "both.c"
    unit.write_text(f'#include "{REF_GPU_H}"\n#include "{os.path.join(ROOT, "include", "gpu.h")}"\n')
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-fsyntax-only", str(unit)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.skipif(not os.path.exists(REF_GPU_H), reason="reference sources absent")
def test_reference_translation_unit_links_and_runs(tmp_path):
    """A C program written against the reference's own include/gpu.h (as
    model.c / inference.c / main.c are) links against libfomoe_gfx950.so with
    every reference function referenced, and its NULL-context calls return the
    reference's "not available" results — host-only, no device is touched."""
    calls = "\n".join(f"    (void)(void *)&{n};" for n in REFERENCE_GPU_H)
    unit = tmp_path / "ref_unit.c"
    unit.write_text(f"""#include <stdio.h>
#include "{REF_GPU_H}"
int main(void) {{
{calls}
    float h[8] = {{0}}, out[8];
    int fails = 0;
    fails += gpu_upload_model(NULL, NULL) != -1;
    fails += gpu_forward(NULL, NULL, 0, 0) != NULL;
    fails += gpu_seed_vram_cache(NULL, NULL, "x") != -1;
    fails += gpu_get_expert_freq(NULL) != NULL;
    fails += gpu_expert_ffn(NULL, h, NULL, NULL, 1, 8, 8, 0, 0, 0, 12, 12, 14, out) != -1;
    int nl = 7, ne = 7;
    gpu_get_expert_dims(NULL, &nl, &ne);
    fails += nl != 0 || ne != 0;
    gpu_register_buffers(NULL, NULL, 0, 0);
    gpu_unregister_buffers(NULL, NULL, 0);
    gpu_set_ram_cache_mb(NULL, 1);
    gpu_set_vram_cache_mb(NULL, 1);
    gpu_reset_state(NULL);
    gpu_enable_expert_freq(NULL);
    gpu_free(NULL);
    printf("fails %d\\n", fails);
    return fails;
}}
""")
    libdir = os.path.dirname(fomoe_amd.LIB_PATH)
    exe = tmp_path / "ref_unit"
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", str(unit), "-o", str(exe), f"-L{libdir}",
                        "-lfomoe_gfx950", f"-Wl,-rpath,{libdir}", "-Wl,-rpath-link,/opt/rocm/lib"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr


def test_reference_lifecycle_stubs_report_not_available():
    """Host-only: the whole-model entry points give the reference's fallback
    answers (no device needed for a NULL context)."""
    lib = fomoe_amd.load_library()
    assert lib.gpu_upload_model(None, None) == -1
    assert lib.gpu_forward(None, None, 0, 0) is None
    assert lib.gpu_seed_vram_cache(None, None, b"x") == -1
    assert lib.gpu_get_expert_freq(None) is None
    nl, ne = C.c_int(7), C.c_int(7)
    lib.gpu_get_expert_dims(None, C.byref(nl), C.byref(ne))
    assert nl.value == 0 and ne.value == 0
    v = [C.c_uint64(9) for _ in range(5)]
    lib.gpu_get_pingpong_relay_stats(None, *[C.byref(x) for x in v])
    assert all(x.value == 0 for x in v)
    lib.gpu_register_buffers(None, None, 0, 0)
    lib.gpu_unregister_buffers(None, None, 0)
    lib.gpu_set_ram_cache_mb(None, 1)
    lib.gpu_set_vram_cache_mb(None, 1)
    lib.gpu_reset_state(None)
    lib.gpu_enable_expert_freq(None)


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
