"""ctypes bindings for the CPU oracle (liboracle.so) and, when built, the
reference CPU library compiled from its own sources (oracle/_ref).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline. The
product package ``fomoe_amd`` never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# ORACLE_LIB: another build of the same restatement (the sanitizer build in tests)
ORACLE_SO = os.environ.get("ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libfomoe_ref.so")

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, BF16, MXFP4 = 0, 1, 8, 12, 13, 14, 30, 39
BLOCK = {Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_0: (32, 34),
         MXFP4: (32, 17), F32: (1, 4), F16: (1, 2), BF16: (1, 2)}
Q8K_BYTES = 4 + 256 + 32  # block_q8_K

_vp, _fp, _ip = C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_int)


def row_bytes(t: int, k: int) -> int:
    vals, nb = BLOCK[t]
    assert k % vals == 0, (t, k)
    return k // vals * nb


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


class MoeDesc(C.Structure):
    _fields_ = [("n_embd", C.c_int), ("inter", C.c_int), ("n_experts", C.c_int), ("k", C.c_int),
                ("gate_type", C.c_int), ("up_type", C.c_int), ("down_type", C.c_int),
                ("gate_size", C.c_uint64), ("up_size", C.c_uint64), ("expert_stride", C.c_uint64),
                ("router", _vp), ("router_bias", _vp), ("experts", _vp), ("shared", _vp),
                ("shared_inter", C.c_int), ("shared_gate_size", C.c_uint64),
                ("shared_up_size", C.c_uint64), ("shared_gate_vec", _vp), ("norm_w", _vp),
                ("eps", C.c_float), ("shared_gate_type", C.c_int), ("shared_up_type", C.c_int),
                ("shared_down_type", C.c_int)]


MOE_NORM, MOE_RESIDUAL = 1, 2


def _load_oracle():
    if not os.path.exists(ORACLE_SO):
        raise RuntimeError(f"{ORACLE_SO} missing: run __graft_entry__.build() (make -C oracle)")
    L = C.CDLL(ORACLE_SO)
    sig = {
        "fo_fp16_to_fp32": (C.c_float, [C.c_uint16]),
        "fo_fp32_to_fp16": (C.c_uint16, [C.c_float]),
        "fo_dequantize_row": (C.c_int, [C.c_int, _vp, _vp, C.c_int64]),
        "fo_vec_dot_f32": (C.c_float, [C.c_int, _vp, _vp, C.c_int64]),
        "fo_mat_vec_mul": (None, [_vp, _vp, C.c_int, _vp, C.c_int64, C.c_int64]),
        "fo_rms_norm": (None, [_vp, _vp, _vp, C.c_int64, C.c_float]),
        "fo_softmax": (None, [_vp, C.c_int64]),
        "fo_silu": (None, [_vp, C.c_int64]),
        "fo_top_k": (None, [_vp, C.c_int64, C.c_int, _vp, _vp]),
        "fo_quantize_row_q8_K": (None, [_vp, _vp, C.c_int64]),
        "fo_matvec_q8": (None, [_vp, _vp, C.c_int, _vp, C.c_int, C.c_int]),
        "fo_cpu_expert_ffn": (None, [_vp, _vp, C.c_float, C.c_int, C.c_int, C.c_int, C.c_uint64,
                                     C.c_uint64, C.c_int, C.c_int, _vp]),
        "fo_moe_layer": (None, [C.POINTER(MoeDesc), _vp, _vp, C.c_int, _vp, _vp]),
        "fo_moe_prefill": (None, [C.POINTER(MoeDesc), _vp, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp]),
        "fo_moe_prefill_w": (None, [C.POINTER(MoeDesc), _vp, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp, C.c_int]),
        "fo_fp32_to_bf16_n": (None, [_vp, _vp, C.c_int64]),
        "fo_rng_key": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "fo_rng_u64": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "fo_normal": (C.c_float, [C.c_uint64, C.c_uint64]),
        "fo_synth_f32": (None, [C.c_uint64, C.c_uint64, C.c_float, _vp, C.c_int64]),
        "fo_quantize": (C.c_int, [C.c_int, _vp, _vp, C.c_int64, C.c_int64]),
        "fo_synth_quant": (C.c_int, [C.c_int, C.c_uint64, C.c_uint64, C.c_float, C.c_int64,
                                     C.c_int64, _vp]),
        "fo_zipf_bias": (None, [C.c_uint64, C.c_uint64, C.c_int, C.c_double, _vp]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    return L


lib = _load_oracle()


# ---------------------------------------------------------------- oracle API
def fp16_to_fp32(h: int) -> float:
    return lib.fo_fp16_to_fp32(h)


def dequantize(t: int, blob: np.ndarray, k: int) -> np.ndarray:
    out = np.empty(k, np.float32)
    assert lib.fo_dequantize_row(t, _ptr(blob), _ptr(out), k) == 0
    return out


def mat_vec(t: int, W: np.ndarray, x: np.ndarray, M: int, K: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(M, np.float32)
    lib.fo_mat_vec_mul(_ptr(out), _ptr(W), t, _ptr(x), M, K)
    return out


def softmax(x: np.ndarray) -> np.ndarray:
    y = np.array(x, np.float32, copy=True)
    lib.fo_softmax(_ptr(y), y.size)
    return y


def top_k(x: np.ndarray, k: int):
    x = np.ascontiguousarray(x, np.float32)
    ids = np.empty(k, np.int32)
    vals = np.empty(k, np.float32)
    lib.fo_top_k(_ptr(x), x.size, k, _ptr(ids), _ptr(vals))
    return ids, vals


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    out = np.empty_like(x, dtype=np.float32)
    lib.fo_rms_norm(_ptr(out), _ptr(np.ascontiguousarray(x, np.float32)),
                    _ptr(np.ascontiguousarray(w, np.float32)), x.size, eps)
    return out


def synth_f32(seed: int, stream: int, std: float, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib.fo_synth_f32(seed, stream, std, _ptr(out), n)
    return out


def quantize(t: int, W: np.ndarray) -> np.ndarray:
    W = np.ascontiguousarray(W, np.float32)
    M, K = W.shape
    out = np.empty(M * row_bytes(t, K), np.uint8)
    assert lib.fo_quantize(t, _ptr(W), _ptr(out), M, K) == 0
    return out


def synth_quant(t: int, seed: int, stream: int, std: float, M: int, K: int) -> np.ndarray:
    out = np.empty(M * row_bytes(t, K), np.uint8)
    assert lib.fo_synth_quant(t, seed, stream, std, M, K, _ptr(out)) == 0
    return out


def zipf_bias(seed: int, stream: int, n: int, s: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib.fo_zipf_bias(seed, stream, n, s, _ptr(out))
    return out


def quantize_q8_K(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size // 256 * Q8K_BYTES, np.uint8)
    lib.fo_quantize_row_q8_K(_ptr(x), _ptr(out), x.size)
    return out


def matvec_q8(t: int, W: np.ndarray, q8: np.ndarray, M: int, K: int) -> np.ndarray:
    out = np.empty(M, np.float32)
    lib.fo_matvec_q8(_ptr(out), _ptr(W), t, _ptr(q8), M, K)
    return out


def cpu_expert_ffn(blob, x, score, gt, ut, dt, gs, us, H, F, partial):
    lib.fo_cpu_expert_ffn(_ptr(blob), _ptr(x), score, gt, ut, dt, gs, us, H, F, _ptr(partial))


def moe_layer(desc: MoeDesc, x: np.ndarray, flags: int):
    out = np.empty(desc.n_embd, np.float32)
    ids = np.empty(desc.k, np.int32)
    w = np.empty(desc.k, np.float32)
    lib.fo_moe_layer(C.byref(desc), _ptr(np.ascontiguousarray(x, np.float32)), _ptr(out), flags,
                     _ptr(ids), _ptr(w))
    return out, ids, w


def to_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (the oracle's rounding)."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib.fo_fp32_to_bf16_n(_ptr(x), _ptr(out), x.size)
    return out


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def moe_prefill(desc: MoeDesc, x_bf16: np.ndarray, t0: int, nt: int, flags: int = 0, bf16_mask: int = 7):
    """Oracle prefill for tokens t0..t0+nt-1 of x_bf16 [T x H] (uint16 bits);
    bf16_mask picks the weight matrices rounded to bf16 (1 gate, 2 up, 4 down);
    8: the down projection on the GPU prefill's fp16 operands instead; 16: the
    choice per expert from its own types, as the GPU prefill makes it."""
    x_bf16 = np.ascontiguousarray(x_bf16, np.uint16)
    H, k = desc.n_embd, desc.k
    out = np.empty((nt, H), np.float32)
    ids = np.empty((nt, k), np.int32)
    w = np.empty((nt, k + 1), np.float32)
    lib.fo_moe_prefill_w(C.byref(desc), _ptr(x_bf16), t0, nt, _ptr(out), flags, _ptr(ids), _ptr(w), bf16_mask)
    return out, ids, w


# ------------------------------------------------- reference library (_ref)
def load_ref():
    """The reference CPU code built from its own sources, or None."""
    if not os.path.exists(REF_SO):
        return None
    R = C.CDLL(REF_SO)
    sig = {
        "fp16_to_fp32": (C.c_float, [C.c_uint16]),
        "fp32_to_fp16": (C.c_uint16, [C.c_float]),
        "dequantize_row_q4_K": (None, [_vp, _vp, C.c_int64]),
        "dequantize_row_q5_K": (None, [_vp, _vp, C.c_int64]),
        "dequantize_row_q6_K": (None, [_vp, _vp, C.c_int64]),
        "dequantize_row_q8_0": (None, [_vp, _vp, C.c_int64]),
        "dequantize_row_mxfp4": (None, [_vp, _vp, C.c_int64]),
        "mat_vec_mul": (None, [_vp, _vp, C.c_int, _vp, C.c_int64, C.c_int64]),
        "mat_vec_mul_fast": (None, [_vp, _vp, C.c_int, _vp, C.c_int, C.c_int]),
        "softmax": (None, [_vp, C.c_int64]),
        "silu": (None, [_vp, C.c_int64]),
        "top_k": (None, [_vp, C.c_int64, C.c_int, _vp, _vp]),
        "rms_norm": (None, [_vp, _vp, _vp, C.c_int64, C.c_float]),
        "quantize_row_q8_K": (None, [_vp, _vp, C.c_int64]),
        "vec_dot_q4_K_q8_K": (C.c_float, [_vp, _vp, C.c_int]),
        "vec_dot_q6_K_q8_K": (C.c_float, [_vp, _vp, C.c_int]),
        "cpu_expert_create": (_vp, [C.c_int, C.c_int]),
        "cpu_expert_free": (None, [_vp]),
        "cpu_expert_reset": (None, [_vp]),
        "cpu_expert_ffn": (None, [_vp, _vp, _vp, C.c_float, C.c_int, C.c_int, C.c_int,
                                  C.c_uint64, C.c_uint64]),
        "cpu_expert_result": (_fp, [_vp]),
    }
    for name, (res, args) in sig.items():
        f = getattr(R, name)
        f.restype, f.argtypes = res, args
    return R
