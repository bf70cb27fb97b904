"""GGUF model files: the library's reader (gpu_gguf_*) against the format of
reference include/gguf.h / src/gguf.c, and resident MoE layers built from a
model's tensors.

CPU: files written by tests/gguf_writer.py read back key by key and tensor by
tensor; the reference's own reader (oracle/_ref: src/gguf.c) agrees on the
same files, split files included; malformed files are rejected. GPU: tensor
uploads (raw and fp32-converted) and gpu_gguf_load_moe_layer's resident
layer run through gpu_moe_layer against the oracle.
"""
import ctypes as C
import os
import struct

import numpy as np
import pytest

import fomoe_amd as FA
import oracle as O
from conftest import inf_rel, parity_err
from gguf_writer import (ARR, BOOL, F32 as VF32, F64, I8, I16, I32, I64, STR, U8, U16, U32, U64,
                         header_bytes, write_gguf)

REF = O.load_ref()
needs_ref = pytest.mark.skipif(REF is None, reason="oracle/_ref not built (reference sources absent)")


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def sample_model():
    """A few keys of every value type and tensors of several ggml types."""
    kvs = [("general.architecture", STR, "qwen35moe"), ("general.name", STR, "tiny test"),
           ("qwen35moe.block_count", U32, 2), ("qwen35moe.expert_used_count", U32, 4),
           ("qwen35moe.attention.layer_norm_rms_epsilon", VF32, 1e-5),
           ("u8", U8, 200), ("i8", I8, -5), ("u16", U16, 60000), ("i16", I16, -30000),
           ("i32", I32, -7), ("u64", U64, 1 << 40), ("i64", I64, -(1 << 40)), ("f64", F64, 0.25),
           ("flag", BOOL, 1), ("arr_i32", ARR, (I32, [1, -2, 3])), ("arr_f32", ARR, (VF32, [0.5, 1.5])),
           ("arr_str", ARR, (STR, ["a", "", "ccc"])), ("arr_empty", ARR, (U8, []))]
    W = O.synth_f32(91, 0, 0.02, 8 * 512).reshape(8, 512)
    tensors = [("vec_f32", [6], FA.F32, O.synth_f32(91, 1, 1.0, 6)),
               ("mat_f16", [5, 3], FA.F16, _f16(O.synth_f32(91, 2, 1.0, 15))),
               ("mat_q4k", [512, 8], FA.Q4_K, O.quantize(O.Q4_K, W)),
               ("mat_q6k", [512, 8], FA.Q6_K, O.quantize(O.Q6_K, W)),
               ("odd_bytes", [7], FA.F16, _f16(np.arange(7)))]
    return kvs, tensors


def test_reader_round_trip(tmp_path):
    kvs, tensors = sample_model()
    p = str(tmp_path / "m.gguf")
    data_off, offs = write_gguf(p, kvs, tensors)
    with FA.Gguf(p) as g:
        assert [k for k, _ in g.keys()] == [k for k, _, _ in kvs]
        assert [t for _, t in g.keys()] == [t for _, t, _ in kvs]
        assert g.get_str("general.architecture") == "qwen35moe"
        assert g.get_int("qwen35moe.expert_used_count") == 4
        assert g.get_int("u8") == 200 and g.get_int("i8") == -5 and g.get_int("u16") == 60000
        assert g.get_int("i16") == -30000 and g.get_int("i32") == -7
        assert g.get_int("u64") == 1 << 40 and g.get_int("i64") == -(1 << 40) and g.get_int("flag") == 1
        assert g.get_float("f64") == 0.25 and g.get_float("i32") == -7.0
        assert abs(g.get_float("qwen35moe.attention.layer_norm_rms_epsilon") - 1e-5) < 1e-12
        assert g.get_int("general.name") is None and g.get_str("u8") is None and g.get_int("nope") is None
        assert list(g.get_arr("arr_i32")) == [1, -2, 3]
        assert list(g.get_arr("arr_f32")) == [0.5, 1.5]
        assert g.get_arr("arr_str") == ["a", "", "ccc"]
        assert g.get_arr("arr_empty").size == 0 and g.get_arr("u8") is None
        ts = g.tensors()
        assert [t["name"] for t in ts] == [t[0] for t in tensors]
        for t, (name, dims, gt, data), off in zip(ts, tensors, offs):
            assert t["dims"] == dims and t["type"] == gt and t["offset"] == off and t["split"] == 0
            assert t["size"] == data.nbytes
            assert g.find_tensor(name) == ts.index(t)
            assert np.array_equal(g.read_tensor(g.find_tensor(name)), data.view(np.uint8))
        assert g.find_tensor("missing") == -1


def test_alignment_key_moves_the_data(tmp_path):
    kvs, tensors = sample_model()
    p = str(tmp_path / "a.gguf")
    write_gguf(p, kvs, tensors, alignment=256)
    with FA.Gguf(p) as g:
        for name, _, _, data in tensors:
            assert np.array_equal(g.read_tensor(g.find_tensor(name)), data.view(np.uint8))
        assert all(t["offset"] % 256 == 0 for t in g.tensors())


def test_type_bytes():
    lib = FA.load_library()
    for t, (vals, nb) in FA.BLOCK.items():
        assert lib.gpu_gguf_type_bytes(t, 10 * vals) == 10 * nb
        assert lib.gpu_gguf_type_bytes(t, 10 * vals + vals // 2) == 10 * nb   # whole blocks only
    assert lib.gpu_gguf_type_bytes(99, 256) == 0


def write_splits(tmp_path, n_write, total=3):
    """Model split over `total` files; only the first n_write are written.
    Split 2 repeats a key with another value (the first file's wins)."""
    parts = []
    for s in range(total):
        kvs = [("split.no", U16, s), ("general.architecture", STR, f"arch{s}")]
        tensors = [(f"t{s}_{j}", [4 * (s + 1)], FA.F32, O.synth_f32(92, 10 * s + j, 1.0, 4 * (s + 1)))
                   for j in range(2)]
        if s == 1:
            kvs.append(("only.in.split2", U32, 42))
        parts.append((kvs, tensors))
    paths = [str(tmp_path / f"model-{s + 1:05d}-of-{total:05d}.gguf") for s in range(total)]
    for s in range(n_write):
        write_gguf(paths[s], *parts[s])
    return paths, parts


@pytest.mark.parametrize("n_write", [3, 2])
def test_split_files_merge(tmp_path, n_write):
    """Splits as in reference src/gguf.c:255-449: tensors appended in split
    order, keys added when new, a missing split skipped."""
    paths, parts = write_splits(tmp_path, n_write)
    with FA.Gguf(paths[0]) as g:
        ts = g.tensors()
        want = [(t[0], s) for s in range(n_write) for t in parts[s][1]]
        assert [(t["name"], t["split"]) for t in ts] == want
        assert g.get_int("split.no") == 0 and g.get_str("general.architecture") == "arch0"
        assert g.get_int("only.in.split2") == 42
        for s in range(n_write):
            for name, _, _, data in parts[s][1]:
                assert np.array_equal(g.read_tensor(g.find_tensor(name)), data.view(np.uint8))


@pytest.mark.parametrize("damage", ["magic", "version1", "version4", "truncated_kv", "truncated_tensors",
                                    "dims", "n_kv", "long_string", "bad_value_type", "missing"])
def test_rejects_malformed_files(tmp_path, damage):
    kvs, tensors = sample_model()
    p = str(tmp_path / "bad.gguf")
    write_gguf(p, kvs, tensors)
    raw = bytearray(open(p, "rb").read())
    hdr, _ = header_bytes(kvs, tensors)
    if damage == "magic":
        raw[0] ^= 0xFF
    elif damage in ("version1", "version4"):
        raw[4:8] = struct.pack("<I", 1 if damage == "version1" else 4)
    elif damage == "truncated_kv":
        raw = raw[:60]
    elif damage == "truncated_tensors":
        raw = raw[:len(hdr) - 10]
    elif damage == "dims":   # first tensor entry claims 5 dims
        i = bytes(raw).index(b"vec_f32") + len(b"vec_f32")
        raw[i:i + 4] = struct.pack("<I", 5)
    elif damage == "n_kv":
        raw[16:24] = struct.pack("<q", 1 << 50)
    elif damage == "long_string":   # first key's length beyond 1 MiB
        raw[24:32] = struct.pack("<Q", (1 << 20) + 1)
    elif damage == "bad_value_type":
        i = 24 + 8 + len("general.architecture")
        raw[i:i + 4] = struct.pack("<i", 77)
    else:
        p = str(tmp_path / "nothing_here.gguf")
    if damage != "missing":
        open(p, "wb").write(bytes(raw))
    with pytest.raises(RuntimeError, match="gguf"):
        FA.Gguf(p)


def test_tensor_past_end_of_file(tmp_path):
    """The directory opens, but a tensor whose data is cut off cannot be read."""
    kvs, tensors = sample_model()
    p = str(tmp_path / "cut.gguf")
    write_gguf(p, kvs, tensors)
    raw = open(p, "rb").read()
    open(p, "wb").write(raw[:len(raw) - 20])
    lib = FA.load_library()
    with FA.Gguf(p) as g:
        last = g.find_tensor("odd_bytes")
        buf = np.empty(64, np.uint8)
        assert lib.gpu_gguf_read_tensor(g.h, last, buf.ctypes.data, buf.size) == -1
        assert np.array_equal(g.read_tensor(g.find_tensor("vec_f32")), tensors[0][3].view(np.uint8))
        assert lib.gpu_gguf_read_tensor(g.h, 0, buf.ctypes.data, 4) == -1      # buffer too small
        assert lib.gpu_gguf_read_tensor(g.h, 99, buf.ctypes.data, 64) == -1    # no such tensor


# ---------------------------------------------------------------- the reference's reader
class RefTensor(C.Structure):
    """gguf_tensor_info_t (reference include/gguf.h:84-92)."""
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_uint32), ("dims", C.c_int64 * 4), ("type", C.c_int),
                ("offset", C.c_uint64), ("size", C.c_uint64), ("split_idx", C.c_int)]


class RefCtx(C.Structure):
    """Leading fields of gguf_ctx_t (reference include/gguf.h:101-114)."""
    _fields_ = [("version", C.c_uint32), ("alignment", C.c_uint64), ("data_offset", C.c_uint64),
                ("n_kv", C.c_int64), ("kv", C.c_void_p), ("n_tensors", C.c_int64),
                ("tensors", C.POINTER(RefTensor))]


def ref_open(path):
    R = REF
    R.gguf_open.restype, R.gguf_open.argtypes = C.POINTER(RefCtx), [C.c_char_p]
    R.gguf_close.argtypes = [C.POINTER(RefCtx)]
    R.gguf_get_u32.restype, R.gguf_get_u32.argtypes = C.c_uint32, [C.POINTER(RefCtx), C.c_char_p]
    R.gguf_get_str.restype, R.gguf_get_str.argtypes = C.c_char_p, [C.POINTER(RefCtx), C.c_char_p]
    R.gguf_find_key.restype, R.gguf_find_key.argtypes = C.c_int64, [C.POINTER(RefCtx), C.c_char_p]
    R.gguf_read_tensor.restype = C.c_size_t
    R.gguf_read_tensor.argtypes = [C.POINTER(RefCtx), C.c_int64, C.c_void_p, C.c_size_t]
    R.gguf_tensor_nbytes.restype, R.gguf_tensor_nbytes.argtypes = C.c_size_t, [C.c_int, C.c_int64]
    return R.gguf_open(path.encode())


@needs_ref
@pytest.mark.parametrize("case", ["single", "aligned", "split"])
def test_agrees_with_reference_reader(tmp_path, monkeypatch, case):
    if case == "split":
        # relative names: the reference looks for "-of-" anywhere in the path
        monkeypatch.chdir(tmp_path)
        paths, _ = write_splits(tmp_path, 3)
        p = os.path.basename(paths[0])
    else:
        kvs, tensors = sample_model()
        p = str(tmp_path / "m.gguf")
        write_gguf(p, kvs, tensors, alignment=64 if case == "aligned" else 32)
    rc = ref_open(p)
    assert rc
    try:
        r = rc.contents
        with FA.Gguf(p) as g:
            ts = g.tensors()
            assert r.n_tensors == len(ts) and r.n_kv == len(g.keys())
            for i, t in enumerate(ts):
                rt = r.tensors[i]
                assert rt.name.decode() == t["name"] and rt.type == t["type"]
                assert list(rt.dims[:rt.n_dims]) == t["dims"]
                assert (rt.offset, rt.size, rt.split_idx) == (t["offset"], t["size"], t["split"])
                buf = np.empty(t["size"], np.uint8)
                assert REF.gguf_read_tensor(rc, i, buf.ctypes.data, buf.size) == t["size"]
                assert np.array_equal(buf, g.read_tensor(i))
            for key, ty in g.keys():
                assert REF.gguf_find_key(rc, key.encode()) >= 0
                if ty == STR:
                    assert REF.gguf_get_str(rc, key.encode()).decode() == g.get_str(key)
                elif ty == U32:
                    assert REF.gguf_get_u32(rc, key.encode()) == g.get_int(key)
        for t in (FA.F32, FA.F16, FA.BF16, FA.Q8_0, FA.Q4_K, FA.Q5_K, FA.Q6_K, FA.MXFP4):
            for n in (256, 4096, 300):
                assert REF.gguf_tensor_nbytes(t, n) == FA.load_library().gpu_gguf_type_bytes(t, n)
    finally:
        REF.gguf_close(rc)


# ---------------------------------------------------------------- GPU: uploads and layers
@pytest.mark.gpu
def test_upload_tensor_and_f32(gpu, tmp_path):
    W = O.synth_f32(93, 0, 0.02, 4 * 512).reshape(4, 512)
    v = O.synth_f32(93, 1, 1.0, 96)
    bf = (v.view(np.uint32) >> 16).astype(np.uint16)
    tensors = [("q4k", [512, 4], FA.Q4_K, O.quantize(O.Q4_K, W)),
               ("q6k", [512, 4], FA.Q6_K, O.quantize(O.Q6_K, W)),
               ("q8_0", [512, 4], FA.Q8_0, O.quantize(O.Q8_0, W)),
               ("f32", [96], FA.F32, v), ("f16", [96], FA.F16, _f16(v)), ("bf16", [96], FA.BF16, bf)]
    p = str(tmp_path / "u.gguf")
    write_gguf(p, [("general.architecture", STR, "x")], tensors)
    with FA.Gguf(p) as g:
        for name, dims, gt, data in tensors:
            i = g.find_tensor(name)
            n = int(np.prod(dims))
            raw = gpu.alloc(data.nbytes)
            gpu.gguf_upload_tensor(g, i, raw, data.nbytes)
            assert np.array_equal(gpu.download(raw, np.uint8, data.nbytes), data.view(np.uint8))
            out = gpu.alloc(4 * n)
            gpu.gguf_upload_f32(g, i, out, n)
            got = gpu.download(out, np.float32, n)
            if gt == FA.F32:
                want = data
            elif gt == FA.F16:
                want = data.view(np.float16).astype(np.float32)
            elif gt == FA.BF16:
                want = (data.astype(np.uint32) << 16).view(np.float32)
            else:
                want = O.dequantize(gt, data, n)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
        with pytest.raises(FA.GpuError, match="elements"):
            gpu.gguf_upload_f32(g, g.find_tensor("f32"), gpu.alloc(4 * 96), 95)


def moe_model(E, H, F, k, seed, down_type=FA.Q6_K, router_type=FA.F32, shared=True, shared_types=None,
              Fs=None, fs_key=None):
    """Tensors of one MoE block (blk.0) in GGUF form and the same weights as
    .qmoe-layout host blobs for the oracle (the shared expert's blob after the
    E routed ones). The shared expert has the routed types and F unless
    shared_types (gate, up, down) / Fs say otherwise; fs_key writes
    {arch}.expert_shared_feed_forward_length."""
    rb_g, rb_d = O.row_bytes(O.Q4_K, H), O.row_bytes(down_type, F)
    st = shared_types or (FA.Q4_K, FA.Q4_K, down_type)
    Fs = Fs or F
    gate = [O.synth_quant(O.Q4_K, seed, 100 + e, 0.02, F, H) for e in range(E)] + \
        [O.synth_quant(st[0], seed, 100 + E, 0.02, Fs, H)]
    up = [O.synth_quant(O.Q4_K, seed, 300 + e, 0.02, F, H) for e in range(E)] + \
        [O.synth_quant(st[1], seed, 300 + E, 0.02, Fs, H)]
    down = [O.synth_quant(down_type, seed, 500 + e, 0.02, H, F) for e in range(E)] + \
        [O.synth_quant(st[2], seed, 500 + E, 0.02, H, Fs)]
    gs, ds = F * rb_g, H * rb_d
    router = O.synth_f32(seed, 1, 0.02, E * H)
    norm = (1.0 + O.synth_f32(seed, 2, 0.1, H)).astype(np.float32)
    gvec = O.synth_f32(seed, 3, 0.05, H)
    if router_type == FA.F16:
        rdata = _f16(router)
        router = rdata.view(np.float16).astype(np.float32)
    else:
        rdata = router
    normbf = (norm.view(np.uint32) >> 16).astype(np.uint16)
    norm = (normbf.astype(np.uint32) << 16).view(np.float32)
    tensors = [("blk.0.ffn_gate_exps.weight", [H, F, E], FA.Q4_K, np.concatenate(gate[:E])),
               ("blk.0.ffn_up_exps.weight", [H, F, E], FA.Q4_K, np.concatenate(up[:E])),
               ("blk.0.ffn_down_exps.weight", [F, H, E], down_type, np.concatenate(down[:E])),
               ("blk.0.ffn_gate_inp.weight", [H, E], router_type, rdata),
               ("blk.0.post_attention_norm.weight", [H], FA.BF16, normbf)]
    if shared:
        tensors += [("blk.0.ffn_gate_shexp.weight", [H, Fs], st[0], gate[E]),
                    ("blk.0.ffn_up_shexp.weight", [H, Fs], st[1], up[E]),
                    ("blk.0.ffn_down_shexp.weight", [Fs, H], st[2], down[E]),
                    ("blk.0.ffn_gate_inp_shexp.weight", [H], FA.F32, gvec)]
    kvs = [("general.architecture", STR, "qwen35moe"), ("qwen35moe.expert_used_count", U32, k),
           ("qwen35moe.attention.layer_norm_rms_epsilon", VF32, 1e-6)]
    if fs_key is not None:
        kvs.append(("qwen35moe.expert_shared_feed_forward_length", U32, fs_key))
    stride = (2 * gs + ds + 4095) // 4096 * 4096
    blobs = np.zeros(E * stride, np.uint8)
    for e in range(E):
        o = e * stride
        blobs[o:o + gs], blobs[o + gs:o + 2 * gs], blobs[o + 2 * gs:o + 2 * gs + ds] = gate[e], up[e], down[e]
    blobs = np.concatenate([blobs, gate[E], up[E], down[E]])
    return kvs, tensors, blobs, gs, ds, stride, router, norm, gvec


SHEXP_CASES = {   # shared expert (gate, up, down) types and F_s differing from the routed Q4_K/Q4_K/down
    "shexp_q6k_down": ((FA.Q4_K, FA.Q4_K, FA.Q6_K), 256),
    "shexp_q8_0_down_fs512": ((FA.Q4_K, FA.Q4_K, FA.Q8_0), 512),
    "shexp_q5k_q8_0_q6k_fs768": ((FA.Q5_K, FA.Q8_0, FA.Q6_K), 768),
}


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["q6k_down_f32_router", "q4k_down_f16_router_no_shared"] + list(SHEXP_CASES))
def test_load_moe_layer_runs_against_oracle(gpu, tmp_path, case):
    """blk.0 of a GGUF model made resident by gpu_gguf_load_moe_layer (expert
    tensors regrouped per expert at the 4096-aligned stride, router / norm /
    shared gate converted to fp32) and run through gpu_moe_layer with norm and
    residual, against the oracle on the same weights (reference
    src/inference.c:481-606). The shexp cases give ffn_*_shexp their own types
    and row count, as the reference reads them (src/model.c:164, 365-371),
    with routed down in Q4_K."""
    E, H, F, k = 12, 512, 256, 4
    dt, rt, shared = (FA.Q6_K, FA.F32, True) if case.startswith("q6k") else (FA.Q4_K, FA.F16, False)
    st, Fs = (FA.Q4_K, FA.Q4_K, dt), F
    if case in SHEXP_CASES:
        (st, Fs), dt, rt, shared = SHEXP_CASES[case], FA.Q4_K, FA.F32, True
    kvs, tensors, blobs, gs, ds, stride, router, norm, gvec = moe_model(
        E, H, F, k, 94, dt, rt, shared, shared_types=st, Fs=Fs, fs_key=Fs if case in SHEXP_CASES else None)
    sgs, sus = O.row_bytes(st[0], H) * Fs, O.row_bytes(st[1], H) * Fs
    p = str(tmp_path / "moe.gguf")
    write_gguf(p, kvs, tensors)
    with FA.Gguf(p) as g:
        L = gpu.gguf_load_moe_layer(g, 0)
    try:
        assert (L.n_embd, L.inter, L.n_experts, L.k) == (H, F, E, k)
        assert (L.gate_type, L.up_type, L.down_type) == (FA.Q4_K, FA.Q4_K, dt)
        assert (L.gate_size, L.up_size, L.expert_stride) == (gs, gs, stride)
        assert abs(L.eps - 1e-6) < 1e-12 and bool(L.shared) == shared and bool(L.shared_gate_vec) == shared
        if shared:
            assert (L.shared_inter, L.shared_gate_size, L.shared_up_size) == (Fs, sgs, sus)
            assert (L.shared_gate_type, L.shared_up_type, L.shared_down_type) == st
            assert np.array_equal(gpu.download(L.shared, np.uint8, blobs.size - E * stride), blobs[E * stride:])
        assert np.array_equal(gpu.download(L.experts, np.uint8, E * stride), blobs[:E * stride])
        assert np.array_equal(gpu.download(L.router, np.float32, E * H), router)
        assert np.array_equal(gpu.download(L.norm_w, np.float32, H), norm)
        x = O.synth_f32(95, 0, 1.0, H)
        dx, dout = gpu.upload(x), gpu.alloc(4 * H)
        gpu.moe_layer(L, dx, dout, FA.MOE_NORM | FA.MOE_RESIDUAL)
        got = gpu.download(dout, np.float32, H)
        d = O.MoeDesc()
        d.n_embd, d.inter, d.n_experts, d.k = H, F, E, k
        d.gate_type, d.up_type, d.down_type = O.Q4_K, O.Q4_K, dt
        d.gate_size, d.up_size, d.expert_stride = gs, gs, stride
        d.router, d.experts = router.ctypes.data, blobs.ctypes.data
        if shared:
            d.shared = blobs.ctypes.data + E * stride
            d.shared_inter, d.shared_gate_size, d.shared_up_size = Fs, sgs, sus
            d.shared_gate_type, d.shared_up_type, d.shared_down_type = st
            d.shared_gate_vec = gvec.ctypes.data
        d.norm_w, d.eps = norm.ctypes.data, 1e-6
        want, ids, w = O.moe_layer(d, x, O.MOE_NORM | O.MOE_RESIDUAL)
        gids, gw, _ = gpu.last_routing(k)
        assert np.array_equal(gids, ids)
        print(f"  gguf layer {case}: parity_err {parity_err(got, want):.3e} inf_rel {inf_rel(got, want):.3e}")
        assert parity_err(got, want) < 1e-3 and inf_rel(got, want) < 1e-5
    finally:
        gpu.gguf_free_moe_layer(L)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["q6k_down_f32_router", "q4k_down_f16_router_no_shared"] + list(SHEXP_CASES))
def test_load_moe_layer_prefill(gpu, tmp_path, case):
    """The GGUF-loaded layer of the cases above through gpu_moe_prefill
    (no RMSNorm; bf16 tokens): routing equal to the oracle's and every token
    against the oracle's composition with each expert's own operand rounding
    (bf16_mask 16); a shared expert whose gate and up are Q5_K and Q8_0 is a
    type mix the prefill does not run (-1)."""
    E, H, F, k, T = 12, 512, 256, 4, 40
    dt, rt, shared = (FA.Q6_K, FA.F32, True) if case.startswith("q6k") else (FA.Q4_K, FA.F16, False)
    st, Fs = (FA.Q4_K, FA.Q4_K, dt), F
    if case in SHEXP_CASES:
        (st, Fs), dt, rt, shared = SHEXP_CASES[case], FA.Q4_K, FA.F32, True
    kvs, tensors, blobs, gs, ds, stride, router, norm, gvec = moe_model(
        E, H, F, k, 94, dt, rt, shared, shared_types=st, Fs=Fs, fs_key=Fs if case in SHEXP_CASES else None)
    sgs, sus = O.row_bytes(st[0], H) * Fs, O.row_bytes(st[1], H) * Fs
    p = str(tmp_path / "moe.gguf")
    write_gguf(p, kvs, tensors)
    with FA.Gguf(p) as g:
        L = gpu.gguf_load_moe_layer(g, 0)
    try:
        x = O.to_bf16(O.synth_f32(96, 0, 1.0, T * H)).reshape(T, H)
        dx, dout = gpu.upload(x), gpu.alloc(4 * T * H)
        if shared and st[0] != st[1] and FA.Q4_K not in st[:2]:
            with pytest.raises(FA.GpuError):
                gpu.moe_prefill(L, dx, T, dout, FA.MOE_RESIDUAL)
            return
        gpu.moe_prefill(L, dx, T, dout, FA.MOE_RESIDUAL)
        got = gpu.download(dout, np.float32, T * H).reshape(T, H)
        ids, w = gpu.prefill_routing(T, k)
        d = O.MoeDesc()
        d.n_embd, d.inter, d.n_experts, d.k = H, F, E, k
        d.gate_type, d.up_type, d.down_type = O.Q4_K, O.Q4_K, dt
        d.gate_size, d.up_size, d.expert_stride = gs, gs, stride
        d.router, d.experts = router.ctypes.data, blobs.ctypes.data
        if shared:
            d.shared = blobs.ctypes.data + E * stride
            d.shared_inter, d.shared_gate_size, d.shared_up_size = Fs, sgs, sus
            d.shared_gate_type, d.shared_up_type, d.shared_down_type = st
            d.shared_gate_vec = gvec.ctypes.data
        want, oids, ow = O.moe_prefill(d, x, 0, T, O.MOE_RESIDUAL, bf16_mask=16)
        assert np.array_equal(ids, oids)
        xf = O.bf16_to_f32(x).reshape(T, H)
        e1 = max(inf_rel(got[t] - xf[t], want[t] - xf[t]) for t in range(T))
        print(f"  gguf prefill {case}: worst token inf_rel (ffn) vs same rounding {e1:.3e}")
        # the prefill's same-rounding bar for its fp16 paths (measured 6.8e-5 with a
        # Q6_K down projection, 5e-6 on the bf16 paths)
        assert e1 <= 3e-4
    finally:
        gpu.gguf_free_moe_layer(L)


@pytest.mark.gpu
def test_load_moe_layer_rejects_bad_models(gpu, tmp_path):
    E, H, F, k = 4, 256, 256, 2
    kvs, tensors, *_ = moe_model(E, H, F, k, 96)
    p = str(tmp_path / "m.gguf")
    write_gguf(p, kvs, tensors)
    with FA.Gguf(p) as g:
        with pytest.raises(FA.GpuError, match="no routed-expert"):
            gpu.gguf_load_moe_layer(g, 1)
    bad = [t if t[0] != "blk.0.ffn_up_exps.weight" else (t[0], [H, F, E - 1], t[2], t[3][:len(t[3]) * (E - 1) // E])
           for t in tensors]
    write_gguf(p, kvs, bad)
    with FA.Gguf(p) as g:
        with pytest.raises(FA.GpuError, match="inconsistent"):
            gpu.gguf_load_moe_layer(g, 0)
    write_gguf(p, [kv for kv in kvs if kv[0] != "qwen35moe.expert_used_count"], tensors)
    with FA.Gguf(p) as g:
        with pytest.raises(FA.GpuError, match="expert_used_count"):
            gpu.gguf_load_moe_layer(g, 0)
    # a shared expert whose row count disagrees with the model's
    # expert_shared_feed_forward_length key
    kvs2, tensors2, *_ = moe_model(E, H, F, k, 96, fs_key=2 * F)
    write_gguf(p, kvs2, tensors2)
    with FA.Gguf(p) as g:
        with pytest.raises(FA.GpuError, match="model key says"):
            gpu.gguf_load_moe_layer(g, 0)
