"""Expert store (.qmoe) ingestion: the file format of reference
include/expert_store.h:8-40 / tools/prepare_experts.c:116-170, read by this
library's host-side index reader and uploaded layer by layer into HBM.

CPU: this module's writer produces the same bytes as the reference's own
writer (oracle/_ref: src/expert_store.c), the library's reader agrees with
the reference's reader, and malformed files are rejected. GPU: a layer
uploaded from a store file runs through gpu_moe_layer against the oracle.
"""
import ctypes as C
import os
import struct

import numpy as np
import pytest

import fomoe_amd as FA
import oracle as O
from conftest import inf_rel, parity_err

ALIGN = 4096
REF = O.load_ref()
needs_ref = pytest.mark.skipif(REF is None, reason="oracle/_ref not built (reference sources absent)")


def align_up(x, a=ALIGN):
    return (x + a - 1) // a * a


def store_layout(n_layers, n_experts, gate_size, up_size, downs):
    """Header fields and index entries the way prepare_experts lays them out:
    stride from the largest down projection, data 4096-aligned after the index."""
    stride = align_up(gate_size + up_size + max(ds for _, ds in downs))
    data_start = align_up(64 + 32 * n_layers)
    entries = [(data_start + l * n_experts * stride, stride, ds, dt) for l, (dt, ds) in enumerate(downs)]
    return stride, entries


def write_qmoe(path, quant_type, gate_size, up_size, downs, blobs):
    """blobs[l][e] = gate|up|down bytes of expert e in layer l."""
    n_layers, n_experts = len(blobs), len(blobs[0])
    stride, entries = store_layout(n_layers, n_experts, gate_size, up_size, downs)
    hdr = struct.pack("<6I4Q8x", 0x454F4D51, 2, n_layers, n_experts, quant_type, ALIGN,
                      gate_size, up_size, max(ds for _, ds in downs), stride)
    idx = b"".join(struct.pack("<3Q2I", off, st, ds, dt, 0) for off, st, ds, dt in entries)
    size = entries[-1][0] + n_experts * stride
    buf = bytearray(size)
    buf[:64] = hdr
    buf[64:64 + len(idx)] = idx
    for l in range(n_layers):
        for e in range(n_experts):
            o = entries[l][0] + e * stride
            buf[o:o + len(blobs[l][e])] = blobs[l][e]
    with open(path, "wb") as f:
        f.write(buf)
    return stride, entries


def make_blobs(n_layers, E, H, F, down_types, seed=61):
    gs = F * O.row_bytes(O.Q4_K, H)
    blobs, downs = [], []
    for l in range(n_layers):
        dt = down_types[l]
        ds = H * O.row_bytes(dt, F)
        downs.append((dt, ds))
        blobs.append([np.concatenate([O.synth_quant(O.Q4_K, seed, (l << 12) | (e << 4) | 0, 0.02, F, H),
                                      O.synth_quant(O.Q4_K, seed, (l << 12) | (e << 4) | 1, 0.02, F, H),
                                      O.synth_quant(dt, seed, (l << 12) | (e << 4) | 2, 0.02, H, F)]).tobytes()
                      for e in range(E)])
    return gs, downs, blobs


class RefHeader(C.Structure):
    _fields_ = [("magic", C.c_uint32), ("version", C.c_uint32), ("n_moe_layers", C.c_uint32),
                ("n_experts", C.c_uint32), ("quant_type", C.c_uint32), ("alignment", C.c_uint32),
                ("expert_gate_size", C.c_uint64), ("expert_up_size", C.c_uint64),
                ("expert_down_size", C.c_uint64), ("expert_stride", C.c_uint64)]


class RefEntry(C.Structure):
    _fields_ = [("data_offset", C.c_uint64), ("expert_stride", C.c_uint64), ("down_size", C.c_uint64),
                ("down_type", C.c_uint32), ("pad", C.c_uint32)]


class RefStore(C.Structure):
    _fields_ = [("fd", C.c_int), ("path", C.c_char_p), ("header", RefHeader),
                ("layer_index", C.POINTER(RefEntry))]


def ref_write(path, quant_type, gate_size, up_size, downs, blobs):
    """The same store written by the reference's expert_store_create / _write_expert."""
    n_layers, n_experts = len(blobs), len(blobs[0])
    stride, entries = store_layout(n_layers, n_experts, gate_size, up_size, downs)
    h = RefHeader(0x454F4D51, 2, n_layers, n_experts, quant_type, ALIGN, gate_size, up_size,
                  max(ds for _, ds in downs), stride)
    ents = (RefEntry * n_layers)(*[RefEntry(o, st, ds, dt, 0) for o, st, ds, dt in entries])
    REF.expert_store_create.restype = C.c_int
    REF.expert_store_create.argtypes = [C.c_char_p, C.c_void_p, C.c_void_p]
    REF.expert_store_write_expert.restype = C.c_bool
    REF.expert_store_write_expert.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_uint64, C.c_void_p, C.c_uint64]
    fd = REF.expert_store_create(path.encode(), C.byref(h), ents)
    assert fd >= 0
    for l in range(n_layers):
        for e in range(n_experts):
            data = np.zeros(stride, np.uint8)
            data[:len(blobs[l][e])] = np.frombuffer(blobs[l][e], np.uint8)
            assert REF.expert_store_write_expert(fd, C.byref(ents[l]), e, stride, data.ctypes.data, stride)
    os.close(fd)


@needs_ref
def test_writer_and_reader_match_reference(tmp_path):
    E, H, F = 5, 256, 256
    gs, downs, blobs = make_blobs(2, E, H, F, [O.Q6_K, O.Q4_K])
    ours, theirs = str(tmp_path / "ours.qmoe"), str(tmp_path / "ref.qmoe")
    stride, entries = write_qmoe(ours, O.Q4_K, gs, gs, downs, blobs)
    ref_write(theirs, O.Q4_K, gs, gs, downs, blobs)
    assert open(ours, "rb").read() == open(theirs, "rb").read()
    # the reference's reader and this library's reader agree
    REF.expert_store_open.restype = C.POINTER(RefStore)
    REF.expert_store_open.argtypes = [C.c_char_p]
    REF.expert_store_offset.restype = C.c_uint64
    REF.expert_store_offset.argtypes = [C.c_void_p, C.c_int, C.c_int]
    st = REF.expert_store_open(theirs.encode())
    assert st
    h, layers = FA.qmoe_read_index(theirs)
    assert (h.n_moe_layers, h.n_experts, h.quant_type, h.expert_stride) == \
        (st.contents.header.n_moe_layers, st.contents.header.n_experts, st.contents.header.quant_type,
         st.contents.header.expert_stride) == (2, E, O.Q4_K, stride)
    for l in range(2):
        r = st.contents.layer_index[l]
        assert (layers[l].data_offset, layers[l].down_size, layers[l].down_type) == \
            (r.data_offset, r.down_size, r.down_type)
        for e in range(E):
            assert REF.expert_store_offset(st, l, e) == layers[l].data_offset + e * layers[l].expert_stride
    REF.expert_store_close.argtypes = [C.c_void_p]
    REF.expert_store_close(st)


def test_read_index_and_layer_desc(tmp_path):
    E, H, F = 4, 256, 256
    gs, downs, blobs = make_blobs(2, E, H, F, [O.Q6_K, O.Q5_K])
    p = str(tmp_path / "s.qmoe")
    stride, entries = write_qmoe(p, O.Q4_K, gs, gs, downs, blobs)
    h, layers = FA.qmoe_read_index(p)
    assert h.magic == FA.C.c_uint32(0x454F4D51).value and h.version == 2
    assert [(L.data_offset, L.expert_stride, L.down_size, L.down_type) for L in layers] == \
        [(o, s, ds, dt) for o, s, ds, dt in entries]
    lib = FA.load_library()
    d = FA.MoeLayer()
    assert lib.gpu_qmoe_layer_desc(C.byref(h), C.byref(layers[1]), C.byref(d)) == 0
    assert (d.gate_type, d.up_type, d.down_type, d.gate_size, d.up_size, d.expert_stride) == \
        (O.Q4_K, O.Q4_K, O.Q5_K, gs, gs, stride)


@pytest.mark.parametrize("damage", ["magic", "version", "truncated", "index"])
def test_rejects_malformed_stores(tmp_path, damage):
    E, H, F = 3, 256, 256
    gs, downs, blobs = make_blobs(1, E, H, F, [O.Q6_K])
    p = str(tmp_path / "bad.qmoe")
    write_qmoe(p, O.Q4_K, gs, gs, downs, blobs)
    raw = bytearray(open(p, "rb").read())
    if damage == "magic":
        raw[0] ^= 0xFF
    elif damage == "version":
        raw[4:8] = struct.pack("<I", 1)
    elif damage == "truncated":
        raw = raw[:len(raw) - 1000]
    else:   # a layer whose stride cannot hold gate + up + down
        raw[64 + 8:64 + 16] = struct.pack("<Q", 4096)
    open(p, "wb").write(bytes(raw))
    with pytest.raises(RuntimeError, match="qmoe"):
        FA.qmoe_read_index(p)


@pytest.mark.gpu
def test_upload_layer_runs_moe_layer(gpu, tmp_path):
    """Layer 1 of a two-layer store (downs Q6_K then Q4_K, stride from the
    larger) uploaded into HBM and run through gpu_moe_layer against the oracle."""
    from test_oracle import moe_desc
    E, H, F, k = 8, 512, 256, 2
    gs, downs, blobs = make_blobs(2, E, H, F, [O.Q6_K, O.Q4_K])
    p = str(tmp_path / "layers.qmoe")
    stride, entries = write_qmoe(p, O.Q4_K, gs, gs, downs, blobs)
    h, layers = FA.qmoe_read_index(p)
    dexp = gpu.alloc(E * stride)
    gpu.qmoe_upload_layer(p, 1, dexp, E * stride)
    raw = open(p, "rb").read()[entries[1][0]:entries[1][0] + E * stride]
    assert np.array_equal(gpu.download(dexp, np.uint8, E * stride), np.frombuffer(raw, np.uint8))
    router = O.synth_f32(62, 3, 0.02, E * H)
    x = O.synth_f32(62, 5, 1.0, H)
    d = FA.MoeLayer()
    d.n_embd, d.inter, d.n_experts, d.k = H, F, E, k
    gpu.qmoe_layer_desc(h, layers[1], d)
    drouter, dx, dout = gpu.upload(router), gpu.upload(x), gpu.alloc(4 * H)
    d.router, d.experts, d.eps = drouter.ptr, dexp.ptr, 1e-6
    gpu.moe_layer(d, dx, dout, 0)
    got = gpu.download(dout, np.float32, H)
    host = np.frombuffer(raw, np.uint8).copy()
    od = moe_desc(E, k, H, F, router, host, gs, downs[1][1])
    od.down_type, od.expert_stride = O.Q4_K, stride
    want, ids, w = O.moe_layer(od, x, 0)
    gids, gw, _ = gpu.last_routing(k)
    assert np.array_equal(gids, ids)
    print(f"  qmoe layer parity_err {parity_err(got, want):.3e} inf_rel {inf_rel(got, want):.3e}")
    assert inf_rel(got, want) < 1e-5
