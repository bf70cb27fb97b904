"""gpu_moe_layer_noalloc (the entry point that allocates nothing) against
gpu_moe_layer, through the C-ABI: the same kernels on a static scratch area,
so the outputs and routing must be bit-identical. Calls in a row on shrinking
layers (the area keeps the previous call's contents), the general (non
three-kernel) path whose router counter must start at zero, and the rejection
of a layer whose scratch exceeds the area. The first call is also checked
against the fp32 oracle (inf_rel < 1e-5, ids equal)."""
import numpy as np
import pytest

import fomoe_amd as FA
import oracle as O
from conftest import inf_rel

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def _layer_pair(gpu, shape, seed, flags, shared_types=None):
    from fomoe_amd import synthetic as S
    L = S.build_layer(gpu, shape, 0, seed=seed, zipf_s=1.1, norm=True)
    if shared_types is not None:   # a shared blob in its own (gate, up, down) types and F_s
        (gt, ut, dt), Fs, H = shared_types[:3], shared_types[3], shape.n_embd
        gs, us, ds = FA.row_bytes(gt, H) * Fs, FA.row_bytes(ut, H) * Fs, FA.row_bytes(dt, Fs) * H
        blob = gpu.alloc(gs + us + ds)
        for t, off, M, K, kind in ((gt, 0, Fs, H, 0), (ut, gs, Fs, H, 1), (dt, gs + us, H, Fs, 2)):
            gpu.synth_quant(t, seed, 900 + kind, 0, 0.02, M, K, 1, blob.offset(off), 0)
        L.buffers.append(blob)
        d = L.desc
        d.shared, d.shared_inter, d.shared_gate_size, d.shared_up_size = blob.ptr, Fs, gs, us
        d.shared_gate_type, d.shared_up_type, d.shared_down_type = gt, ut, dt
    x = O.synth_f32(seed + 1, 0, 1.0, shape.n_embd)
    dx = gpu.upload(x)
    ref, got = gpu.alloc(4 * shape.n_embd), gpu.alloc(4 * shape.n_embd)
    gpu.moe_layer(L.desc, dx, ref, flags)
    ids_a, w_a, sw_a = gpu.last_routing(shape.k)
    rc = gpu.moe_layer_noalloc(L.desc, dx, got, flags)
    assert rc == 0, gpu.last_error()
    ids_b, w_b, sw_b = gpu.last_routing(shape.k)
    a = gpu.download(ref, np.float32, shape.n_embd)
    b = gpu.download(got, np.float32, shape.n_embd)
    assert np.array_equal(ids_a, ids_b)
    assert np.array_equal(w_a.view(np.uint32), w_b.view(np.uint32)) and sw_a == sw_b
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return L, x, b, ids_b, w_b


def test_noalloc_matches_moe_layer_on_consecutive_calls(gpu):
    from fomoe_amd import synthetic as S
    from test_oracle import moe_desc
    # call 1: config-3 expert shape on 64 experts (three-kernel path), norm + residual
    shape = S.LayerShape(n_embd=4096, inter=1024, n_experts=64, k=10)
    say("noalloc call 1", shape)
    L, x, out, ids, w = _layer_pair(gpu, shape, 51, FA.MOE_NORM | FA.MOE_RESIDUAL)
    E, H, F, k = shape.n_experts, shape.n_embd, shape.inter, shape.k
    router = O.synth_f32(51, S.stream(0, 0, S.ROUTER), 0.02, E * H)
    bias = O.zipf_bias(51, S.stream(0, 0, S.ZIPF), E, 1.1)
    experts = np.zeros((E + 1) * shape.stride, np.uint8)
    for e in [int(v) for v in ids] + [E]:
        b = np.concatenate([O.synth_quant(O.Q4_K, 51, S.stream(0, e, S.GATE), 0.02, F, H),
                            O.synth_quant(O.Q4_K, 51, S.stream(0, e, S.UP), 0.02, F, H),
                            O.synth_quant(O.Q6_K, 51, S.stream(0, e, S.DOWN), 0.02, H, F)])
        experts[e * shape.stride:e * shape.stride + b.size] = b
    norm_w = np.ones(H, np.float32)
    d = moe_desc(E, k, H, F, router, experts, shape.gate_size, shape.down_size,
                 shared_off=E * shape.stride, bias=bias, norm_w=norm_w)
    d.expert_stride = shape.stride
    want, oid, _ = O.moe_layer(d, x, O.MOE_NORM | O.MOE_RESIDUAL)
    assert np.array_equal(ids, oid)
    say(f"  inf_rel vs oracle {inf_rel(out, want):.3e}")
    assert inf_rel(out, want) < 1e-5
    del L
    # call 2: a smaller layer right after (three-kernel path, no shared expert)
    shape = S.LayerShape(n_embd=1024, inter=512, n_experts=16, k=4, shared=False)
    say("noalloc call 2", shape)
    _layer_pair(gpu, shape, 52, 0)
    # call 3: smaller still, on the general path (n_embd not a multiple of 512)
    shape = S.LayerShape(n_embd=768, inter=256, n_experts=8, k=2)
    say("noalloc call 3", shape)
    _layer_pair(gpu, shape, 53, FA.MOE_NORM)


@pytest.mark.parametrize("st", [((FA.Q4_K, FA.Q4_K, FA.Q8_0), 1024), ((FA.Q5_K, FA.Q4_K, FA.Q8_0), 512)])
def test_noalloc_shared_expert_own_types(gpu, st):
    """A shared expert whose down type alone differs (its block in the
    reduce kernel) and one in types and F_s of its own (the fp32 shared-expert
    kernels): the no-allocation call stays bit-identical to gpu_moe_layer,
    twice in a row."""
    from fomoe_amd import synthetic as S
    shape = S.LayerShape(n_embd=4096, inter=1024, n_experts=32, k=8)
    say("noalloc shared own types", st)
    for seed in (81, 82):
        _layer_pair(gpu, shape, seed, FA.MOE_NORM | FA.MOE_RESIDUAL, shared_types=(*st[0], st[1]))


@pytest.mark.parametrize("down,st", [(FA.Q5_K, None), (FA.Q4_K, None),
                                     (FA.Q5_K, ((FA.Q4_K, FA.Q4_K, FA.Q6_K), 1024))])
def test_noalloc_down_groups_of_32(gpu, down, st):
    """Q5_K / Q4_K routed down projections at the config shape (the gate/up
    kernel leaves fp32 activations in the area, the down kernel prepares its
    32-value groups from them), alone and with a Q6_K shared down block:
    bit-identical to gpu_moe_layer, twice in a row."""
    from fomoe_amd import synthetic as S
    shape = S.LayerShape(n_embd=4096, inter=1024, n_experts=32, k=8, down_type=down)
    say("noalloc down groups of 32", down, st)
    for seed in (83, 84):
        _layer_pair(gpu, shape, seed, FA.MOE_NORM | FA.MOE_RESIDUAL,
                    shared_types=None if st is None else (*st[0], st[1]))


def test_noalloc_rejects_layers_beyond_the_area(gpu):
    """H = F = 8192 with 16 + 1 experts needs ~1.1 MB of scratch: -1 and a
    message, before any device work (the descriptor's pointers are never read)."""
    dummy = gpu.alloc(4096)
    L = FA.MoeLayer()
    L.n_embd, L.inter, L.n_experts, L.k = 8192, 8192, 64, 16
    L.gate_type = L.up_type = FA.Q4_K
    L.down_type = FA.Q6_K
    L.gate_size = L.up_size = 8192 * FA.row_bytes(FA.Q4_K, 8192)
    L.expert_stride = 2 * L.gate_size + 8192 * FA.row_bytes(FA.Q6_K, 8192)
    L.router, L.experts, L.shared = dummy.ptr, dummy.ptr, dummy.ptr
    L.shared_inter, L.shared_gate_size, L.shared_up_size, L.eps = 8192, L.gate_size, L.gate_size, 1e-6
    L.shared_gate_type, L.shared_up_type, L.shared_down_type = FA.Q4_K, FA.Q4_K, FA.Q6_K
    out = gpu.alloc(4 * 8192)
    assert gpu.moe_layer_noalloc(L, out, out, 0) == -1
    assert "scratch" in gpu.last_error()
