"""GPU parity of benchmark config 4 at its real size: the 60-layer, 512-expert,
top-10, Zipf(1.1)-routed Q4_K/Q6_K stack, fully HBM-resident (251.6 GB),
decoded from the captured HIP graph of gpu_moe_stack_decode.

Per layer the stack computes x <- x + moe(rms_norm(x)) (reference
src/inference.c:481-606 with the residual of inference.c:606). Checks:
- the graph-replayed stack (two decode steps) is bit-identical to the same 120
  layer calls issued one by one through gpu_moe_layer, whose inputs and
  routing are recorded;
- at sampled layers (first, middle, last of the first step) the routing ids
  equal the oracle's, the layer output is within inf_rel 1e-5 of the fp32
  oracle (oracle.c fo_moe_layer) on the GPU's own input, and the layer's
  increment (output - input) is within parity_err 1e-3 of the exact layer
  (fp64 rms_norm, router, softmax and renormalised weights over the same
  dequantized experts).
Only the sampled layers' router and selected experts are rebuilt on the CPU
(bit-identical generator, checked on the downloaded bytes).
"""
import numpy as np
import pytest

import oracle as O
from conftest import inf_rel, parity_err

pytestmark = pytest.mark.gpu

N_LAYERS = 60
SAMPLED = (0, 29, 59)


def say(*a):
    print(*a, flush=True)


def _exact_increment(x, router, bias, ids, blobs, shape):
    """fp64 ffn of one layer for input x (no residual), routing by `ids`."""
    E, H, F, k = shape.n_experts, shape.n_embd, shape.inter, shape.k
    x64 = x.astype(np.float64)
    hn = x64 / np.sqrt((x64 * x64).mean() + 1e-6)
    lg = router.astype(np.float64).reshape(E, H) @ hn + bias.astype(np.float64)
    p = np.exp(lg - lg.max())
    p /= p.sum()
    w = p[ids] / p[ids].sum()
    out = np.zeros(H)
    for r, e in enumerate(list(ids) + [E]):
        g_b, u_b, d_b = blobs[int(e)]
        G = O.dequantize(O.Q4_K, g_b, F * H).reshape(F, H).astype(np.float64)
        U = O.dequantize(O.Q4_K, u_b, F * H).reshape(F, H).astype(np.float64)
        D = O.dequantize(O.Q6_K, d_b, H * F).reshape(H, F).astype(np.float64)
        g = G @ hn
        out += (float(w[r]) if r < k else 1.0) * (D @ (g / (1 + np.exp(-g)) * (U @ hn)))
    return out


def test_stack_config4_full(gpu):
    from fomoe_amd import synthetic as S
    from test_oracle import moe_desc
    shape = S.LayerShape()
    E, H, F, k, stride = shape.n_experts, shape.n_embd, shape.inter, shape.k, shape.stride
    need = N_LAYERS * ((E + 1) * stride + 4 * E * H)
    if gpu.hbm < need + (8 << 30):
        pytest.skip(f"config 4 needs {need / 1e9:.1f} GB resident, device has {gpu.hbm / 1e9:.1f} GB")
    say(f"stack config4: building {N_LAYERS} layers ({need / 1e9:.1f} GB)")
    layers = []
    try:
        for l in range(N_LAYERS):
            layers.append(S.build_layer(gpu, shape, l, seed=4, zipf_s=1.1))
        gpu.sync()
        descs = [L.desc for L in layers]
        x0 = O.synth_f32(4, S.stream(0, 0, S.HIDDEN), 1.0, H)
        # the captured stack, two steps
        dx = gpu.upload(x0)
        say("stack config4: graph decode, 2 steps")
        gpu.stack_decode(descs, dx, 2)
        gpu.sync()
        x_graph = gpu.download(dx, np.float32, H)
        # the same 120 layer calls one by one, recording the first step
        say("stack config4: layer by layer, 2 steps")
        dy = gpu.upload(x0)
        inputs, routing = [x0.copy()], {}
        for step in range(2):
            for l in range(N_LAYERS):
                gpu.moe_layer(descs[l], dy, dy, O.MOE_NORM | O.MOE_RESIDUAL)
                if step == 0:
                    if l in SAMPLED:
                        routing[l] = gpu.last_routing(k)
                    inputs.append(gpu.download(dy, np.float32, H))
        x_calls = gpu.download(dy, np.float32, H)
        say(f"stack config4: final x rms {np.sqrt((x_graph.astype(np.float64) ** 2).mean()):.3f}")
        assert np.isfinite(x_graph).all()
        assert np.array_equal(x_graph.view(np.uint32), x_calls.view(np.uint32))
        for l in SAMPLED:
            xin, xout = inputs[l], inputs[l + 1]
            ids, w, _ = routing[l]
            router = O.synth_f32(4, S.stream(l, 0, S.ROUTER), 0.02, E * H)
            bias = O.zipf_bias(4, S.stream(l, 0, S.ZIPF), E, 1.1)
            norm_w = np.ones(H, np.float32)
            hn = O.rms_norm(xin, norm_w, 1e-6)
            lg = O.mat_vec(O.F32, router, hn, E, H) + bias
            oi, _ = O.top_k(O.softmax(lg.astype(np.float32)), k)
            assert np.array_equal(ids, oi), (l, ids, oi)
            table = np.zeros((E + 1) * stride, np.uint8)
            blobs = {}
            for e in [int(v) for v in oi] + [E]:
                blobs[e] = (O.synth_quant(O.Q4_K, 4, S.stream(l, e, S.GATE), 0.02, F, H),
                            O.synth_quant(O.Q4_K, 4, S.stream(l, e, S.UP), 0.02, F, H),
                            O.synth_quant(O.Q6_K, 4, S.stream(l, e, S.DOWN), 0.02, H, F))
                blob = np.concatenate(blobs[e])
                dev = gpu.download(descs[l].experts + e * stride, np.uint8, blob.size)
                assert np.array_equal(dev, blob), (l, e)
                table[e * stride:e * stride + blob.size] = blob
            d = moe_desc(E, k, H, F, router, table, shape.gate_size, shape.down_size,
                         shared_off=E * stride, bias=bias, norm_w=norm_w)
            d.expert_stride = stride
            want, _, ow = O.moe_layer(d, xin, O.MOE_NORM | O.MOE_RESIDUAL)
            inc = xout.astype(np.float64) - xin.astype(np.float64)
            exact = _exact_increment(xin, router, bias, oi, blobs, shape)
            e_par, e_rel = parity_err(inc, exact), inf_rel(xout, want)
            say(f"  PARITY config4 layer {l}: ids {list(ids)} increment parity_err(exact) {e_par:.3e} "
                f"output inf_rel(fp32 oracle) {e_rel:.3e} weights inf_rel {inf_rel(w, ow):.3e}")
            assert inf_rel(w, ow) < 1e-5
            assert e_rel < 1e-5
            assert e_par <= 1e-3
    finally:
        for L in layers:
            for b in L.buffers:
                b.free()
