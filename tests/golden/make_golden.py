"""Write tests/golden/golden.npz from the REFERENCE CPU code.

The reference library is compiled from the reference's own sources
(src/quant.c, src/tensor.c, src/gguf.c, src/cpu_expert.c) by oracle/Makefile
into oracle/_ref/libfomoe_ref.so; this script calls it on seeded inputs and
stores inputs (or the seeds + SHA-256 of inputs that the oracle's generator
reproduces) together with the reference outputs. Run in the build container:

    make -C oracle && python tests/golden/make_golden.py

The fixture is data only (inputs and expected outputs); no reference source
is copied.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")


def P(a):
    return a.ctypes.data_as(C.c_void_p)


def sha(a: np.ndarray) -> np.ndarray:
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), np.uint8)


def random_blocks(rng, t, nblocks):
    vals, bb = O.BLOCK[t]
    raw = rng.integers(0, 256, size=nblocks * bb, dtype=np.uint8)
    b = raw.reshape(nblocks, bb)
    # keep the fp16 scale fields finite (exponent != 31) so outputs compare
    def finite(col):
        hi = b[:, col]
        bad = (hi & 0x7C) == 0x7C
        hi[bad] &= 0xBF
        b[:, col] = hi
    if t in (O.Q4_K, O.Q5_K):
        finite(1); finite(3)
    elif t == O.Q6_K:
        finite(209)
    elif t == O.Q8_0:
        finite(1)
    return raw


def main():
    R = O.load_ref()
    if R is None:
        sys.exit("oracle/_ref/libfomoe_ref.so missing: run make -C oracle (needs /root/reference)")
    rng = np.random.default_rng(20261201)
    g = {}
    deq = {O.Q4_K: R.dequantize_row_q4_K, O.Q5_K: R.dequantize_row_q5_K,
           O.Q6_K: R.dequantize_row_q6_K, O.Q8_0: R.dequantize_row_q8_0,
           O.MXFP4: R.dequantize_row_mxfp4}
    # ---- dequantization of random blocks (every bit pattern of every field)
    for t, fn in deq.items():
        vals, bb = O.BLOCK[t]
        nb = 96
        raw = random_blocks(rng, t, nb)
        y = np.empty(nb * vals, np.float32)
        fn(P(raw), P(y), nb * vals)
        g[f"deq_{t}_in"] = raw
        g[f"deq_{t}_out"] = y
    # ---- mat_vec_mul (fp32 activations) on synthetic quantized rows
    for t, (M, K) in {O.Q4_K: (16, 4096), O.Q5_K: (8, 1024), O.Q6_K: (16, 1024),
                      O.Q8_0: (16, 1024)}.items():
        W = O.synth_quant(t, 100 + t, 7, 0.02, M, K)
        x = O.synth_f32(200 + t, 7, 1.0, K)
        y = np.empty(M, np.float32)
        R.mat_vec_mul(P(y), P(W), t, P(x), M, K)
        g[f"mv_{t}_W"], g[f"mv_{t}_x"], g[f"mv_{t}_y"] = W, x, y
    # F32 router-shaped matvec
    Wf = O.synth_f32(300, 7, 0.02, 64 * 512)
    xf = O.synth_f32(301, 7, 1.0, 512)
    yf = np.empty(64, np.float32)
    R.mat_vec_mul(P(yf), P(Wf), O.F32, P(xf), 64, 512)
    g["mv_f32_seed"] = np.array([300, 301, 7, 64, 512], np.int64)
    g["mv_f32_in_sha"] = sha(np.concatenate([Wf, xf]))
    g["mv_f32_y"] = yf
    # ---- softmax / top_k (with exact ties) / rms_norm
    lg = rng.standard_normal(512).astype(np.float32)
    lg[[3, 77, 300]] = lg.max() + 1.0          # a three-way tie at the top
    lg[[10, 11]] = np.float32(lg.max() - 0.5)  # and another tie
    sm = lg.copy()
    R.softmax(P(sm), sm.size)
    ids = np.empty(10, np.int32)
    vals = np.empty(10, np.float32)
    R.top_k(P(sm), sm.size, 10, P(ids), P(vals))
    g["softmax_in"], g["softmax_out"], g["topk_ids"], g["topk_vals"] = lg, sm, ids, vals
    xr = rng.standard_normal(4096).astype(np.float32) * 3
    wr = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    outr = np.empty(4096, np.float32)
    R.rms_norm(P(outr), P(xr), P(wr), 4096, np.float32(1e-6))
    g["rms_x"], g["rms_w"], g["rms_out"] = xr, wr, outr
    # ---- Q8_K quantization and integer dots (cpu_expert baseline path)
    xq = O.synth_f32(400, 7, 1.0, 4096)
    q8 = np.zeros(16 * O.Q8K_BYTES, np.uint8)
    R.quantize_row_q8_K(P(xq), P(q8), 4096)
    W4 = O.synth_quant(O.Q4_K, 401, 7, 0.02, 4, 4096)
    W6 = O.synth_quant(O.Q6_K, 402, 7, 0.02, 4, 4096)
    d4 = np.array([R.vec_dot_q4_K_q8_K(P(W4[r * 2304:]), P(q8), 16) for r in range(4)], np.float32)
    d6 = np.array([R.vec_dot_q6_K_q8_K(P(W6[r * 3360:]), P(q8), 16) for r in range(4)], np.float32)
    g["q8k_x"], g["q8k_out"], g["q8k_W4"], g["q8k_W6"] = xq, q8, W4, W6
    g["q8k_dot4"], g["q8k_dot6"] = d4, d6
    # ---- cpu_expert engine: one expert, reduced shape
    H, F = 512, 256
    gs = F * O.row_bytes(O.Q4_K, H)
    ds = H * O.row_bytes(O.Q6_K, F)
    blob = np.concatenate([O.synth_quant(O.Q4_K, 500, 1, 0.02, F, H),
                           O.synth_quant(O.Q4_K, 500, 2, 0.02, F, H),
                           O.synth_quant(O.Q6_K, 500, 3, 0.02, H, F)])
    xin = O.synth_f32(501, 7, 1.0, H)
    ce = R.cpu_expert_create(H, F)
    R.cpu_expert_reset(ce)
    R.cpu_expert_ffn(ce, P(blob), P(xin), np.float32(0.75), O.Q4_K, O.Q4_K, O.Q6_K, gs, gs)
    part = np.ctypeslib.as_array(R.cpu_expert_result(ce), shape=(H,)).copy()
    R.cpu_expert_free(ce)
    g["cpuexp_seed"] = np.array([500, 501, H, F], np.int64)
    g["cpuexp_in_sha"] = sha(np.concatenate([blob.view(np.uint8), xin.view(np.uint8)]))
    g["cpuexp_out"] = part
    assert ds + 2 * gs == blob.size
    # ---- MoE layer composed from the reference CPU functions in the order
    # of reference src/inference.c:484-596 (reduced shape, seeded inputs)
    E, k, H, F = 16, 4, 512, 256
    router = O.synth_f32(600, 3, 0.02, E * H)
    h = O.synth_f32(600, 5, 1.0, H)
    stride = 2 * gs + ds
    experts = np.concatenate([np.concatenate([O.synth_quant(O.Q4_K, 600, (e << 4) | 0, 0.02, F, H),
                                              O.synth_quant(O.Q4_K, 600, (e << 4) | 1, 0.02, F, H),
                                              O.synth_quant(O.Q6_K, 600, (e << 4) | 2, 0.02, H, F)])
                              for e in range(E + 1)])  # expert E = shared
    logits = np.empty(E, np.float32)
    R.mat_vec_mul(P(logits), P(router), O.F32, P(h), E, H)
    R.softmax(P(logits), E)
    sel = np.empty(k, np.int32)
    sv = np.empty(k, np.float32)
    R.top_k(P(logits), E, k, P(sel), P(sv))
    ssum = np.float32(0)
    for i in range(k):
        ssum = np.float32(ssum + sv[i])
    sv = (sv * np.float32(np.float32(1) / ssum)).astype(np.float32)

    def ffn(off):
        gb = np.empty(F, np.float32)
        ub = np.empty(F, np.float32)
        db = np.empty(H, np.float32)
        e = experts[off:]
        R.mat_vec_mul(P(gb), P(e), O.Q4_K, P(h), F, H)
        R.silu(P(gb), F)
        R.mat_vec_mul(P(ub), P(e[gs:]), O.Q4_K, P(h), F, H)
        gb = (gb * ub).astype(np.float32)
        R.mat_vec_mul(P(db), P(e[2 * gs:]), O.Q6_K, P(gb), H, F)
        return db

    out = np.zeros(H, np.float32)
    for i in range(k):
        out = (out + sv[i] * ffn(int(sel[i]) * stride)).astype(np.float32)
    out = (out + ffn(E * stride)).astype(np.float32)
    g["moe_seed"] = np.array([600, E, k, H, F], np.int64)
    g["moe_in_sha"] = sha(np.concatenate([router.view(np.uint8), h.view(np.uint8), experts]))
    g["moe_ids"], g["moe_w"], g["moe_out"] = sel, sv, out
    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(g)} arrays)")


if __name__ == "__main__":
    main()
