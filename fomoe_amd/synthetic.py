"""Device-resident synthetic workloads of the benchmark configurations.

Stream numbering (this build's own definition; the reference has no
synthetic data): stream(layer, expert, kind) = ((layer + 1) << 24) |
(expert << 4) | kind, with expert == n_experts naming the shared expert and
kind GATE 0, UP 1, DOWN 2, ROUTER 3, HIDDEN 5, ZIPF 6 (router bias), TOKENS 7
(prefill activations). Weights are N(0, 0.02) fp32
quantized by this build's quantizers; activations N(0, 1). Every byte is
generated on the device by libfomoe_gfx950 (bit-identical to oracle/'s CPU
generator, which the tests use to check samples).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import Q4_K, Q6_K, Gpu, MoeLayer, row_bytes

GATE, UP, DOWN, ROUTER, HIDDEN, ZIPF, TOKENS = 0, 1, 2, 3, 5, 6, 7
W_STD = 0.02


def stream(layer: int, expert: int, kind: int) -> int:
    return ((layer + 1) << 24) | (expert << 4) | kind


@dataclass
class LayerShape:
    n_embd: int = 4096
    inter: int = 1024
    n_experts: int = 512
    k: int = 10
    gate_type: int = Q4_K
    down_type: int = Q6_K
    shared: bool = True

    @property
    def gate_size(self) -> int:
        return self.inter * row_bytes(self.gate_type, self.n_embd)

    @property
    def down_size(self) -> int:
        return self.n_embd * row_bytes(self.down_type, self.inter)

    @property
    def stride(self) -> int:
        s = 2 * self.gate_size + self.down_size
        return (s + 4095) // 4096 * 4096   # expert blobs on 4 KiB boundaries

    def expert_bytes(self) -> int:
        """Algorithmic bytes of one expert (gate + up + down)."""
        return 2 * self.gate_size + self.down_size


@dataclass
class DeviceLayer:
    desc: MoeLayer
    buffers: list = field(default_factory=list)


def build_layer(gpu: Gpu, shape: LayerShape, layer: int, seed: int = 4,
                zipf_s: float | None = None, norm: bool = True) -> DeviceLayer:
    """One MoE layer's router, experts and shared expert, generated in HBM."""
    s = shape
    E, H, F = s.n_experts, s.n_embd, s.inter
    n_blobs = E + (1 if s.shared else 0)
    experts = gpu.alloc(n_blobs * s.stride)
    for kind, off, t, M, K in ((GATE, 0, s.gate_type, F, H), (UP, s.gate_size, s.gate_type, F, H),
                               (DOWN, 2 * s.gate_size, s.down_type, H, F)):
        gpu.synth_quant(t, seed, stream(layer, 0, kind), 16, W_STD, M, K, n_blobs,
                        experts.offset(off), s.stride)
    router = gpu.alloc(4 * E * H)
    gpu.synth_f32(seed, stream(layer, 0, ROUTER), W_STD, router, E * H)
    bufs = [experts, router]
    bias = None
    if zipf_s is not None:
        bias = gpu.upload(gpu.zipf_bias(seed, stream(layer, 0, ZIPF), E, zipf_s))
        bufs.append(bias)
    norm_w = None
    if norm:
        norm_w = gpu.upload(np.ones(H, np.float32))
        bufs.append(norm_w)
    d = MoeLayer()
    d.n_embd, d.inter, d.n_experts, d.k = H, F, E, s.k
    d.gate_type, d.up_type, d.down_type = s.gate_type, s.gate_type, s.down_type
    d.gate_size, d.up_size, d.expert_stride = s.gate_size, s.gate_size, s.stride
    d.router, d.router_bias = router.ptr, (bias.ptr if bias else None)
    d.experts = experts.ptr
    d.shared = experts.offset(E * s.stride) if s.shared else None
    d.shared_inter, d.shared_gate_size, d.shared_up_size = F, s.gate_size, s.gate_size
    d.shared_gate_type, d.shared_up_type, d.shared_down_type = s.gate_type, s.gate_type, s.down_type
    d.shared_gate_vec = None
    d.norm_w = norm_w.ptr if norm_w else None
    d.eps = 1e-6
    return DeviceLayer(d, bufs)


def hidden(gpu: Gpu, n_embd: int, seed: int = 4):
    """The layer input h ~ N(0, 1) (config 3)."""
    buf = gpu.alloc(4 * n_embd)
    gpu.synth_f32(seed, stream(0, 0, HIDDEN), 1.0, buf, n_embd)
    return buf


def tokens_bf16(gpu: Gpu, n_tokens: int, n_embd: int, seed: int = 4):
    """Prefill activations X [n_tokens x n_embd] ~ N(0, 1), rounded to bf16
    (config 5); returns the bf16 device buffer."""
    n = n_tokens * n_embd
    tmp = gpu.alloc(4 * n)
    gpu.synth_f32(seed, stream(0, 0, TOKENS), 1.0, tmp, n)
    x = gpu.alloc(2 * n)
    gpu.f32_to_bf16(tmp, x, n)
    gpu.sync()
    tmp.free()
    return x
