"""Pins of the CPU oracle (oracle/oracle.c) — CPU only.

Each function of the oracle is checked against (a) the committed golden
fixtures written by the reference's own code (tests/golden/make_golden.py),
(b) the reference library compiled from its sources (oracle/_ref) when it is
present, and (c) what the mathematics fixes independently of both: IEEE
binary16 via numpy, exactness of the dequantization products, fp64 dots,
softmax/top-k properties, quantizer error bounds.
"""
import ctypes as C
import hashlib
import os

import numpy as np
import pytest

import oracle as O
from conftest import inf_rel, parity_err

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
REF = O.load_ref()
needs_ref = pytest.mark.skipif(REF is None, reason="oracle/_ref not built (reference sources absent)")


def P(a):
    return a.ctypes.data_as(C.c_void_p)


def sha(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), np.uint8)


# ------------------------------------------------------------------ fp16
def test_fp16_to_fp32_exhaustive_vs_ieee():
    codes = np.arange(65536, dtype=np.uint32)
    got = np.array([O.lib.fo_fp16_to_fp32(int(h)) for h in codes], np.float32)
    ieee = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ieee)
    assert np.array_equal(got[~nan].view(np.uint32), ieee[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()


def test_fp32_to_fp16_rne_vs_ieee():
    rng = np.random.default_rng(1)
    bits = np.concatenate([rng.integers(0, 2**32, 400000, dtype=np.uint64).astype(np.uint32),
                           # the binary16 range edges, subnormals and halfway cases
                           np.arange(0x33000000, 0x33000000 + 20000, dtype=np.uint32),
                           np.arange(0x387FE000, 0x38802000, dtype=np.uint32),
                           np.arange(0x477FE000, 0x47800400, dtype=np.uint32)])
    f = bits.view(np.float32)
    f = f[~np.isnan(f)]
    got = np.array([O.lib.fo_fp32_to_fp16(float(v)) for v in f], np.uint16)
    with np.errstate(over="ignore"):
        ieee = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ieee)
    assert O.lib.fo_fp32_to_fp16(float("nan")) & 0x7FFF == 0x7E00


@needs_ref
def test_fp16_conversions_vs_reference():
    for h in list(range(0, 65536, 7)) + [0x7C00, 0xFC00, 0x0001, 0x03FF, 0x0400]:
        a, b = O.lib.fo_fp16_to_fp32(h), REF.fp16_to_fp32(h)
        assert (a == b) or (np.isnan(a) and np.isnan(b))
    rng = np.random.default_rng(2)
    for v in rng.standard_normal(20000).astype(np.float32) * np.float32(1e3):
        assert O.lib.fo_fp32_to_fp16(float(v)) == REF.fp32_to_fp16(float(v))


# ------------------------------------------------------------------ dequant
@pytest.mark.parametrize("t", [O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0, O.MXFP4])
def test_dequant_golden_bit_exact(t):
    raw, want = GOLD[f"deq_{t}_in"], GOLD[f"deq_{t}_out"]
    got = O.dequantize(t, raw, want.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("t", [O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0])
def test_dequant_synth_vs_reference(t):
    W = O.synth_quant(t, 11, 3, 0.02, 32, 1024)
    got = O.dequantize(t, W, 32 * 1024)
    want = np.empty_like(got)
    fn = {O.Q4_K: REF.dequantize_row_q4_K, O.Q5_K: REF.dequantize_row_q5_K,
          O.Q6_K: REF.dequantize_row_q6_K, O.Q8_0: REF.dequantize_row_q8_0}[t]
    fn(P(W), P(want), got.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _q4k_block(d, dmin, sc, m, q):
    """Pack one Q4_K block from field values, following the GGUF layout."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    for j in range(4):
        b[4 + j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        b[8 + j] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        b[12 + j] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    for g in range(4):
        for l in range(32):
            b[16 + 32 * g + l] = q[64 * g + l] | (q[64 * g + 32 + l] << 4)
    return b


def test_q4k_brute_force_all_scale_min_codes():
    """Every (6-bit scale, 6-bit min) pair in every sub-block position, every
    nibble: y = fl(d*sc*q - dmin*m) with both products exact (closed form)."""
    rng = np.random.default_rng(3)
    blocks, want = [], []
    pairs = [(s, m) for s in range(64) for m in range(64)]
    for i in range(0, len(pairs), 8):
        sc = np.array([p[0] for p in pairs[i:i + 8]], np.int64)
        mm = np.array([p[1] for p in pairs[i:i + 8]], np.int64)
        q = rng.integers(0, 16, 256)
        q[:16] = np.arange(16)
        d, dmin = np.float16(rng.uniform(1e-4, 0.01)), np.float16(rng.uniform(1e-4, 0.01))
        blocks.append(_q4k_block(d, dmin, sc, mm, q))
        sub = np.arange(256) // 32
        exact = np.float64(d) * sc[sub] * q - np.float64(dmin) * mm[sub]
        want.append(exact.astype(np.float32))  # one rounding of the exact value
    got = O.dequantize(O.Q4_K, np.concatenate(blocks), 256 * len(blocks))
    assert np.array_equal(got, np.concatenate(want))


def test_q6k_closed_form_all_codes():
    """Q6_K: y = d*sc*(q-32), exact for every 6-bit code and every int8 scale."""
    rng = np.random.default_rng(4)
    for trial in range(16):
        u = rng.integers(0, 64, 256)
        u[:64] = np.arange(64)
        sc = rng.integers(-128, 128, 16)
        sc[trial % 16] = -128
        d = np.float16(rng.uniform(1e-5, 1e-2))
        b = np.zeros(210, np.uint8)
        for n in range(2):
            for l in range(32):
                e = 128 * n + l
                q1, q2, q3, q4 = u[e], u[e + 32], u[e + 64], u[e + 96]
                b[64 * n + l] = (q1 & 15) | ((q3 & 15) << 4)
                b[64 * n + l + 32] = (q2 & 15) | ((q4 & 15) << 4)
                b[128 + 32 * n + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
        b[192:208] = sc.astype(np.int8).view(np.uint8)
        b[208:210] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
        got = O.dequantize(O.Q6_K, b, 256)
        want = (np.float64(d) * sc[np.arange(256) // 16] * (u - 32)).astype(np.float32)
        assert np.array_equal(got, want)


def test_q8_0_and_mxfp4_closed_form():
    rng = np.random.default_rng(5)
    b = np.zeros(34 * 8, np.uint8).reshape(8, 34)
    q = rng.integers(-128, 128, (8, 32))
    ds = [np.float16(v) for v in rng.uniform(-0.1, 0.1, 8)]
    for i in range(8):
        b[i, :2] = np.frombuffer(ds[i].tobytes(), np.uint8)
        b[i, 2:] = q[i].astype(np.int8).view(np.uint8)
    got = O.dequantize(O.Q8_0, b.ravel(), 256)
    want = np.concatenate([(np.float64(ds[i]) * q[i]).astype(np.float32) for i in range(8)])
    assert np.array_equal(got, want)
    e2m1 = [0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6]
    mb = np.zeros(17, np.uint8)
    mb[0] = 130
    mb[1:] = np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4)
    got = O.dequantize(O.MXFP4, mb, 32)
    want = np.array([e2m1[c] * 8 for c in range(16)] + [e2m1[15 - c] * 8 for c in range(16)], np.float32)
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ matvec
@pytest.mark.parametrize("t", [O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0])
def test_matvec_golden(t):
    W, x, y = GOLD[f"mv_{t}_W"], GOLD[f"mv_{t}_x"], GOLD[f"mv_{t}_y"]
    K = x.size
    got = O.mat_vec(t, W, x, y.size, K)
    # the reference build contracts with FMA, the oracle does not: fp32 reordering only
    assert inf_rel(got, y) < 1e-5
    # and the inputs are what the oracle's generator makes for these seeds
    assert np.array_equal(W, O.synth_quant(t, 100 + t, 7, 0.02, y.size, K))
    # fp64 dot of the (bit-exact) dequantized rows
    deq = O.dequantize(t, W, y.size * K).reshape(y.size, K).astype(np.float64)
    assert inf_rel(got, deq @ x.astype(np.float64)) < 1e-5


def test_matvec_f32_golden():
    s = GOLD["mv_f32_seed"]
    Wf = O.synth_f32(int(s[0]), int(s[2]), 0.02, int(s[3] * s[4]))
    xf = O.synth_f32(int(s[1]), int(s[2]), 1.0, int(s[4]))
    assert np.array_equal(sha(np.concatenate([Wf, xf])), GOLD["mv_f32_in_sha"])
    got = O.mat_vec(O.F32, Wf, xf, int(s[3]), int(s[4]))
    assert inf_rel(got, GOLD["mv_f32_y"]) < 1e-5


# ------------------------------------------------------------------ softmax / top-k / norm
def test_softmax_topk_golden_bit_exact():
    sm = O.softmax(GOLD["softmax_in"])
    assert np.array_equal(sm, GOLD["softmax_out"])
    ids, vals = O.top_k(sm, 10)
    assert np.array_equal(ids, GOLD["topk_ids"]) and np.array_equal(vals, GOLD["topk_vals"])
    # ties resolve to the lowest index, values non-increasing
    assert list(ids[:3]) == [3, 77, 300] and list(ids[3:5]) == [10, 11]
    assert np.all(np.diff(vals) <= 0)


def test_softmax_topk_properties():
    rng = np.random.default_rng(6)
    x = rng.standard_normal(512).astype(np.float32) * 3
    sm = O.softmax(x)
    ref = np.exp(x.astype(np.float64) - x.max())
    ref /= ref.sum()
    assert inf_rel(sm, ref) < 1e-5
    ids, vals = O.top_k(sm, 10)
    order = np.lexsort((np.arange(512), -sm))  # descending value, ascending index
    assert np.array_equal(ids, order[:10])


def test_rms_norm_golden():
    got = O.rms_norm(GOLD["rms_x"], GOLD["rms_w"], 1e-6)
    assert inf_rel(got, GOLD["rms_out"]) < 1e-6


# ------------------------------------------------------------------ Q8_K baseline path
def test_q8k_quantize_golden_bit_exact():
    got = O.quantize_q8_K(GOLD["q8k_x"])
    assert np.array_equal(got, GOLD["q8k_out"])


def test_q8k_dots_golden():
    q8 = GOLD["q8k_out"]
    d4 = O.matvec_q8(O.Q4_K, GOLD["q8k_W4"], q8, 4, 4096)
    d6 = O.matvec_q8(O.Q6_K, GOLD["q8k_W6"], q8, 4, 4096)
    assert inf_rel(d4, GOLD["q8k_dot4"]) < 1e-5
    assert inf_rel(d6, GOLD["q8k_dot6"]) < 1e-5


def test_cpu_expert_golden():
    s = GOLD["cpuexp_seed"]
    H, F = int(s[2]), int(s[3])
    gs = F * O.row_bytes(O.Q4_K, H)
    blob = np.concatenate([O.synth_quant(O.Q4_K, int(s[0]), 1, 0.02, F, H),
                           O.synth_quant(O.Q4_K, int(s[0]), 2, 0.02, F, H),
                           O.synth_quant(O.Q6_K, int(s[0]), 3, 0.02, H, F)])
    xin = O.synth_f32(int(s[1]), 7, 1.0, H)
    assert np.array_equal(sha(np.concatenate([blob, xin.view(np.uint8)])), GOLD["cpuexp_in_sha"])
    part = np.zeros(H, np.float32)
    O.cpu_expert_ffn(blob, xin, 0.75, O.Q4_K, O.Q4_K, O.Q6_K, gs, gs, H, F, part)
    assert inf_rel(part, GOLD["cpuexp_out"]) < 1e-4


# ------------------------------------------------------------------ MoE composition
def _moe_inputs(seed, E, H, F):
    gs = F * O.row_bytes(O.Q4_K, H)
    ds = H * O.row_bytes(O.Q6_K, F)
    router = O.synth_f32(seed, 3, 0.02, E * H)
    h = O.synth_f32(seed, 5, 1.0, H)
    experts = np.concatenate([np.concatenate([O.synth_quant(O.Q4_K, seed, (e << 4) | 0, 0.02, F, H),
                                              O.synth_quant(O.Q4_K, seed, (e << 4) | 1, 0.02, F, H),
                                              O.synth_quant(O.Q6_K, seed, (e << 4) | 2, 0.02, H, F)])
                              for e in range(E + 1)])
    return router, h, experts, gs, ds


def moe_desc(E, k, H, F, router, experts, gs, ds, shared_off=None, bias=None, norm_w=None, gvec=None):
    d = O.MoeDesc()
    d.n_embd, d.inter, d.n_experts, d.k = H, F, E, k
    d.gate_type, d.up_type, d.down_type = O.Q4_K, O.Q4_K, O.Q6_K
    d.gate_size, d.up_size, d.expert_stride = gs, gs, 2 * gs + ds
    d.router = router.ctypes.data
    d.router_bias = bias.ctypes.data if bias is not None else None
    d.experts = experts.ctypes.data
    d.shared = experts.ctypes.data + shared_off if shared_off is not None else None
    d.shared_inter, d.shared_gate_size, d.shared_up_size = F, gs, gs
    d.shared_gate_type, d.shared_up_type, d.shared_down_type = O.Q4_K, O.Q4_K, O.Q6_K
    d.shared_gate_vec = gvec.ctypes.data if gvec is not None else None
    d.norm_w = norm_w.ctypes.data if norm_w is not None else None
    d.eps = 1e-6
    return d


def test_moe_layer_golden():
    s = GOLD["moe_seed"]
    seed, E, k, H, F = (int(v) for v in s)
    router, h, experts, gs, ds = _moe_inputs(seed, E, H, F)
    assert np.array_equal(sha(np.concatenate([router.view(np.uint8), h.view(np.uint8), experts])),
                          GOLD["moe_in_sha"])
    d = moe_desc(E, k, H, F, router, experts, gs, ds, shared_off=E * (2 * gs + ds))
    out, ids, w = O.moe_layer(d, h, 0)
    assert np.array_equal(ids, GOLD["moe_ids"])
    assert inf_rel(w, GOLD["moe_w"]) < 1e-6
    assert parity_err(out, GOLD["moe_out"]) < 1e-4


def test_moe_layer_fp64_recomposition():
    """The oracle's layer equals an fp64 recomposition from dequantized weights."""
    E, k, H, F = 8, 3, 256, 256
    router, h, experts, gs, ds = _moe_inputs(77, E, H, F)
    stride = 2 * gs + ds
    norm_w = np.ones(H, np.float32) * np.float32(1.5)
    gvec = O.synth_f32(78, 0, 0.05, H)
    d = moe_desc(E, k, H, F, router, experts, gs, ds, shared_off=E * stride, norm_w=norm_w, gvec=gvec)
    out, ids, w = O.moe_layer(d, h, O.MOE_NORM | O.MOE_RESIDUAL)
    x = h.astype(np.float64)
    hn = x / np.sqrt((x * x).mean() + 1e-6) * 1.5
    logits = router.reshape(E, H).astype(np.float64) @ hn
    p = np.exp(logits - logits.max())
    p /= p.sum()
    sel = np.lexsort((np.arange(E), -p))[:k]
    assert np.array_equal(ids, sel)
    wt = p[sel] / p[sel].sum()

    def ffn(off):
        e = experts[off:off + stride]
        G = O.dequantize(O.Q4_K, e[:gs], F * H).reshape(F, H).astype(np.float64)
        U = O.dequantize(O.Q4_K, e[gs:2 * gs], F * H).reshape(F, H).astype(np.float64)
        D = O.dequantize(O.Q6_K, e[2 * gs:], H * F).reshape(H, F).astype(np.float64)
        g = G @ hn
        return D @ (g / (1 + np.exp(-g)) * (U @ hn))

    ref = sum(wt[i] * ffn(int(sel[i]) * stride) for i in range(k))
    ref = ref + ffn(E * stride) / (1 + np.exp(-(hn @ gvec.astype(np.float64))))
    assert parity_err(out, x + ref) < 1e-4


@pytest.mark.parametrize("Fs,st", [(512, (O.Q8_0, O.Q5_K, O.Q6_K)), (256, (O.Q6_K, O.Q4_K, O.Q8_0))])
def test_moe_layer_shared_own_types_fp64(Fs, st):
    """A shared expert in its own tensor types and intermediate size
    (reference include/model.h:104-108, src/inference.c:361-374): the oracle's
    layer equals an fp64 recomposition, and handing it the routed types
    instead changes the output (the types are really read)."""
    E, k, H, F = 8, 3, 256, 256
    router, h, experts, gs, ds = _moe_inputs(79, E, H, F)
    stride = 2 * gs + ds
    sh = [O.synth_quant(st[0], 80, 0, 0.02, Fs, H), O.synth_quant(st[1], 80, 1, 0.02, Fs, H),
          O.synth_quant(st[2], 80, 2, 0.02, H, Fs)]
    table = np.concatenate([experts[:E * stride]] + sh)
    d = moe_desc(E, k, H, F, router, table, gs, ds, shared_off=E * stride)
    d.shared_inter, d.shared_gate_size, d.shared_up_size = Fs, sh[0].size, sh[1].size
    d.shared_gate_type, d.shared_up_type, d.shared_down_type = st
    out, ids, w = O.moe_layer(d, h, 0)
    hn = h.astype(np.float64)

    def ffn(types, mats, Fe):
        G, U, D = (O.dequantize(t, m, r * c).reshape(r, c).astype(np.float64)
                   for t, m, r, c in zip(types, mats, (Fe, Fe, H), (H, H, Fe)))
        g = G @ hn
        return D @ (g / (1 + np.exp(-g)) * (U @ hn))

    routed = [(experts[e * stride:e * stride + gs], experts[e * stride + gs:e * stride + 2 * gs],
               experts[e * stride + 2 * gs:(e + 1) * stride]) for e in ids]
    lg = router.reshape(E, H).astype(np.float64) @ hn
    p = np.exp(lg - lg.max())
    wt = p[ids] / p[ids].sum()
    ref = sum(wt[i] * ffn((O.Q4_K, O.Q4_K, O.Q6_K), routed[i], F) for i in range(k)) + ffn(st, sh, Fs)
    # the fp32 oracle's own sequential sums: 1.1e-4 measured at the 1e-3 floor
    assert parity_err(out, ref) < 3e-4
    d.shared_gate_type, d.shared_up_type, d.shared_down_type = O.Q4_K, O.Q4_K, O.Q6_K
    d.shared_inter = min(Fs, F)
    wrong, _, _ = O.moe_layer(d, h, 0)
    assert not parity_err(wrong, ref) <= 1e-2   # (NaN too: other bytes read as fp16 scales)


# ------------------------------------------------------------------ synthetic generator
def test_normal_generator_statistics():
    z = O.synth_f32(5, 0, 1.0, 1 << 20).astype(np.float64)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1) < 3e-3
    assert abs((z ** 3).mean()) < 2e-2 and abs((z ** 4).mean() - 3) < 3e-2
    # pairs are (r cos t, r sin t): r^2 = -2 ln u1 ~ Exp(1/2)
    r2 = z[0::2] ** 2 + z[1::2] ** 2
    assert abs(r2.mean() - 2) < 2e-2
    # deterministic and stream-separated
    assert np.array_equal(O.synth_f32(5, 0, 1.0, 1000), O.synth_f32(5, 0, 1.0, 1000))
    assert not np.array_equal(O.synth_f32(5, 1, 1.0, 1000), O.synth_f32(5, 0, 1.0, 1000))


@pytest.mark.parametrize("t,maxrel", [(O.Q4_K, 0.09), (O.Q5_K, 0.045), (O.Q6_K, 0.02), (O.Q8_0, 0.005)])
def test_quantizer_round_trip(t, maxrel):
    W = O.synth_f32(9, 1, 0.02, 64 * 1024).reshape(64, 1024)
    q = O.quantize(t, W)
    back = O.dequantize(t, q, W.size).reshape(W.shape)
    # error bounded by a fraction of each row's range, and unbiased
    rng = np.abs(W).max(axis=1, keepdims=True)
    assert (np.abs(back - W) / rng).max() < maxrel
    assert abs(float((back - W).mean())) < 1e-5
    corr = np.corrcoef(back.ravel(), W.ravel())[0, 1]
    assert corr > {O.Q4_K: 0.99, O.Q5_K: 0.997, O.Q6_K: 0.999, O.Q8_0: 0.9999}[t]


def test_zipf_bias_is_a_permuted_log_rank():
    b = O.zipf_bias(4, 6, 512, 1.1)
    r = np.sort(-b / 1.1)
    assert np.allclose(np.exp(r), np.arange(1, 513), rtol=1e-5)
    assert not np.array_equal(np.argsort(-b)[:10], np.arange(10))


# ------------------------------------------------------------------ bf16 / prefill
def test_bf16_rounding_vs_torch():
    """fp32 -> bf16 round-to-nearest-even equals torch's conversion, including
    exact halfway cases, subnormals, infinities and the largest finite values."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    half = (rng.integers(0, 1 << 16, 4096, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000
    x = np.concatenate([bits, half, np.array([0x7F7FFFFF, 0xFF7FFFFF, 0x00008000, 0x00018000,
                                              0x7F800000, 0xFF800000], np.uint32)]).view(np.float32)
    x = x[np.isfinite(x) | np.isinf(x)]
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.to_bf16(x), ref)


def _prefill_inputs(seed, E, H, F, T):
    router, _, experts, gs, ds = _moe_inputs(seed, E, H, F)
    x = O.to_bf16(O.synth_f32(seed, 9, 1.0, T * H)).reshape(T, H)
    return router, x, experts, gs, ds


def _q6k_f16_operands(blob, rows, cols):
    """Q6_K rows as the fp16 down operands: fp16(q - 32) * fp16(d * sc), each
    product rounded to fp16; value order of reference src/quant.c:147-175,
    parsed here independently of the oracle's C code."""
    b = np.frombuffer(blob, np.uint8).reshape(-1, 210)
    ql, qh = b[:, :128].astype(np.int32), b[:, 128:192].astype(np.int32)
    sc = b[:, 192:208].view(np.int8).astype(np.float32)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    e = np.arange(256)
    n, t, l = e >> 7, (e & 127) >> 5, e & 31
    qlb = ql[:, 64 * n + l + 32 * (t & 1)]
    lo = np.where(t & 2, qlb >> 4, qlb & 15)
    hi = (qh[:, 32 * n + l] >> (2 * t)) & 3
    q = (lo | (hi << 4)) - 32
    dsc = (d[:, None] * sc).astype(np.float16).astype(np.float32)[:, e >> 4]
    w = (q.astype(np.float32) * dsc).astype(np.float16).astype(np.float32)
    return w.reshape(rows, cols)


def _act_f16(a):
    """fp16 activation row with its power-of-two scale: v = hi + lo (bf16
    split), max|v| brought into [2^14, 2^15)."""
    a = np.asarray(a, np.float32)
    hi = O.bf16_to_f32(O.to_bf16(a))
    v = hi + O.bf16_to_f32(O.to_bf16(a - hi))
    s = int(np.frexp(np.float32(np.abs(v).max()))[1]) - 15
    return np.ldexp(v, -s).astype(np.float16).astype(np.float64), s


@pytest.mark.parametrize("mask", [7, 4, 0, 8])
def test_prefill_oracle_fp64_recomposition(mask):
    """Prefill oracle = numpy recomposition: exact dequantized weights, rounded
    to bf16 for the matrices in bf16_mask (1 gate, 2 up, 4 down), fp64 dots,
    fp32 SwiGLU activation, rank-order combine; mask 8: the Q6_K down
    projection on fp16 operands (weights fp16(q - 32) * fp16(d * sc), the
    activation as fp16 under its row's power-of-two scale)."""
    E, k, H, F, T = 8, 3, 256, 256, 5
    router, x, experts, gs, ds = _prefill_inputs(41, E, H, F, T)
    stride = 2 * gs + ds
    gvec = O.synth_f32(42, 0, 0.05, H)
    d = moe_desc(E, k, H, F, router, experts, gs, ds, shared_off=E * stride, gvec=gvec)
    out, ids, w = O.moe_prefill(d, x, 1, 3, O.MOE_RESIDUAL, bf16_mask=mask)

    def bfm(a, bit):   # bf16-rounded when the matrix's bit is in the mask
        return (O.bf16_to_f32(O.to_bf16(a)) if mask & bit else a).astype(np.float64)

    def ffn(off, xt):
        e = experts[off:off + stride]
        G = bfm(O.dequantize(O.Q4_K, e[:gs], F * H), 1).reshape(F, H)
        U = bfm(O.dequantize(O.Q4_K, e[gs:2 * gs], F * H), 2).reshape(F, H)
        g, u = (G @ xt).astype(np.float32), (U @ xt).astype(np.float32)
        a = (g / (1 + np.exp(-g))) * u
        if mask & 8:
            D = _q6k_f16_operands(e[2 * gs:], H, F).astype(np.float64)
            a16, sx = _act_f16(a)
            return np.ldexp(D @ a16, sx)
        D = bfm(O.dequantize(O.Q6_K, e[2 * gs:], H * F), 4).reshape(H, F)
        return D @ a.astype(np.float64)

    for i, t in enumerate(range(1, 4)):
        xt = O.bf16_to_f32(x[t]).astype(np.float64)
        logits = router.reshape(E, H).astype(np.float64) @ xt
        p = np.exp(logits - logits.max())
        p /= p.sum()
        sel = np.lexsort((np.arange(E), -p))[:k]
        assert np.array_equal(ids[i], sel)
        wt = p[sel] / p[sel].sum()
        assert inf_rel(w[i, :k], wt) < 1e-5
        sg = 1 / (1 + np.exp(-(xt @ gvec.astype(np.float64))))
        assert abs(w[i, k] - sg) < 1e-6
        ref = sum(wt[j] * ffn(int(sel[j]) * stride, xt) for j in range(k)) + sg * ffn(E * stride, xt)
        # mask 8: an fp32 SwiGLU value one ulp apart (numpy vs C expf) can round
        # to the neighbouring fp16, 2^-11 of one term
        assert parity_err(out[i], xt + ref) < (1e-4 if mask & 8 else 1e-5)


def _q8_0_f16_operands(blob, rows, cols):
    """Q8_0 rows as the fp16 down operands: fp16(d * q), the product rounded
    once; block layout of reference src/quant.c:266-274 (fp16 d, 32 int8),
    parsed here independently of the oracle's C code."""
    b = np.frombuffer(blob, np.uint8).reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)[:, 0]
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d[:, None] * q).astype(np.float16).astype(np.float32).reshape(rows, cols)


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4_K, O.Q5_K])
def test_prefill_oracle_fp16_down_types(dt):
    """Prefill oracle with a Q8_0 / Q4_K / Q5_K down projection on fp16
    operands (mask 8, and the per-expert rule of mask 16) = numpy
    recomposition: exact Q4_K gate/up; down weights fp16(d * q) (Q8_0, parsed
    here) or the exact dequantized value rounded to fp16 (Q4_K, Q5_K); the
    activation as fp16 under its row's power of two."""
    E, k, H, F, T = 6, 2, 256, 256, 3
    router = O.synth_f32(44, 0, 0.02, E * H)
    gs, ds = O.row_bytes(O.Q4_K, H) * F, O.row_bytes(dt, F) * H
    stride = 2 * gs + ds
    experts = np.concatenate([np.concatenate([O.synth_quant(O.Q4_K, 45, 3 * e, 0.02, F, H),
                                              O.synth_quant(O.Q4_K, 45, 3 * e + 1, 0.02, F, H),
                                              O.synth_quant(dt, 45, 3 * e + 2, 0.02, H, F)]) for e in range(E)])
    x = O.to_bf16(O.synth_f32(46, 0, 1.0, T * H)).reshape(T, H)
    d = moe_desc(E, k, H, F, router, experts, gs, ds)
    d.down_type = dt
    for mask in (8, 16):
        out, ids, w = O.moe_prefill(d, x, 0, T, 0, bf16_mask=mask)
        for t in range(T):
            xt = O.bf16_to_f32(x[t]).astype(np.float64)
            ref = np.zeros(H)
            for j in range(k):
                e = experts[int(ids[t, j]) * stride:(int(ids[t, j]) + 1) * stride]
                G = O.dequantize(O.Q4_K, e[:gs], F * H).reshape(F, H).astype(np.float64)
                U = O.dequantize(O.Q4_K, e[gs:2 * gs], F * H).reshape(F, H).astype(np.float64)
                g, u = (G @ xt).astype(np.float32), (U @ xt).astype(np.float32)
                a16, sx = _act_f16((g / (1 + np.exp(-g))) * u)
                if dt == O.Q8_0:
                    D = _q8_0_f16_operands(e[2 * gs:], H, F).astype(np.float64)
                else:
                    D = O.dequantize(dt, e[2 * gs:], H * F).reshape(H, F).astype(np.float16).astype(np.float64)
                ref += float(w[t, j]) * np.ldexp(D @ a16, sx)
            # an fp32 SwiGLU value one ulp apart (numpy vs C expf) can round to
            # the neighbouring fp16, 2^-11 of one term
            assert parity_err(out[t], ref) < 1e-4, (mask, t)


def test_prefill_oracle_close_to_fp32_layer():
    """bf16 weights/activations move the prefill output by ~1e-3 of its scale
    from the fp32 decode oracle on the same (bf16) input; routing identical."""
    E, k, H, F, T = 8, 3, 512, 256, 4
    router, x, experts, gs, ds = _prefill_inputs(43, E, H, F, T)
    d = moe_desc(E, k, H, F, router, experts, gs, ds, shared_off=E * (2 * gs + ds))
    out, ids, w = O.moe_prefill(d, x, 0, T, 0)
    for t in range(T):
        ref, rids, rw = O.moe_layer(d, O.bf16_to_f32(x[t]), 0)
        assert np.array_equal(ids[t], rids)
        assert inf_rel(w[t, :k], rw) < 1e-6
        assert inf_rel(out[t], ref) < 2e-2
