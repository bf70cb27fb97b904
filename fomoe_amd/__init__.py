"""fomoe_amd — MI355X (gfx950) quantized MoE expert hot path.

Python binding of libfomoe_gfx950.so through its C-ABI (include/gpu.h). The
library is the product: every computation below runs in its HIP kernels. If
the library is missing the import fails loudly — there is no CPU fallback.

Device buffers are plain device pointers owned by :class:`DeviceBuffer`.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# FOMOE_LIB: another build of the same library (the host-sanitizer build in
# tests); the product library otherwise.
LIB_PATH = os.environ.get("FOMOE_LIB") or os.path.join(HERE, "libfomoe_gfx950.so")

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, BF16, MXFP4 = 0, 1, 8, 12, 13, 14, 30, 39
BLOCK = {Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_0: (32, 34),
         MXFP4: (32, 17), F32: (1, 4), F16: (1, 2), BF16: (1, 2)}
MOE_NORM, MOE_RESIDUAL = 1, 2

_vp = C.c_void_p

# Every symbol include/gpu.h declares, with its ctypes signature.
SIGNATURES = {
    "gpu_init": (_vp, []),
    "gpu_free": (None, [_vp]),
    "gpu_expert_ffn": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_uint64,
                                 C.c_uint64, C.c_uint64, C.c_int, C.c_int, C.c_int, _vp]),
    "gpu_register_buffers": (None, [_vp, _vp, C.c_int, C.c_uint64]),
    "gpu_unregister_buffers": (None, [_vp, _vp, C.c_int]),
    "gpu_upload_model": (C.c_int, [_vp, _vp]),
    "gpu_set_ram_cache_mb": (None, [_vp, C.c_int]),
    "gpu_set_vram_cache_mb": (None, [_vp, C.c_int]),
    "gpu_forward": (_vp, [_vp, _vp, C.c_int, C.c_int]),
    "gpu_reset_state": (None, [_vp]),
    "gpu_seed_vram_cache": (C.c_int, [_vp, _vp, C.c_char_p]),
    "gpu_enable_expert_freq": (None, [_vp]),
    "gpu_get_expert_freq": (_vp, [_vp]),
    "gpu_get_expert_dims": (None, [_vp, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "gpu_get_pingpong_relay_stats": (None, [_vp] + [C.POINTER(C.c_uint64)] * 5),
    "gpu_alloc": (_vp, [_vp, C.c_uint64]),
    "gpu_dealloc": (None, [_vp, _vp]),
    "gpu_upload": (C.c_int, [_vp, _vp, _vp, C.c_uint64]),
    "gpu_download": (C.c_int, [_vp, _vp, _vp, C.c_uint64]),
    "gpu_sync": (C.c_int, [_vp]),
    "gpu_device_info": (C.c_int, [_vp, C.POINTER(C.c_int), C.POINTER(C.c_uint64), C.c_char_p, C.c_int]),
    "gpu_last_error": (C.c_char_p, [_vp]),
    "gpu_dequantize": (C.c_int, [_vp, C.c_int, _vp, _vp, C.c_int64]),
    "gpu_matvec_q": (C.c_int, [_vp, C.c_int, _vp, _vp, _vp, C.c_int, C.c_int]),
    "gpu_matvec_q_batched": (C.c_int, [_vp, C.c_int, _vp, C.c_uint64, C.c_int, _vp, C.c_uint64,
                                       _vp, C.c_uint64, C.c_int, C.c_int]),
    "gpu_moe_layer": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int]),
    "gpu_moe_layer_noalloc": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int]),
    "gpu_moe_last_routing": (C.c_int, [_vp, _vp, _vp, _vp]),
    "gpu_router_topk": (C.c_int, [_vp, _vp, _vp, _vp, _vp, C.c_float, C.c_int, C.c_int, C.c_int,
                                  _vp, _vp]),
    "gpu_moe_stack_decode": (C.c_int, [_vp, _vp, C.c_int, _vp, C.c_int]),
    "gpu_qmoe_read_index": (C.c_int, [C.c_char_p, _vp, _vp, C.c_int, C.POINTER(C.c_char_p)]),
    "gpu_qmoe_upload_layer": (C.c_int, [_vp, C.c_char_p, C.c_int, _vp, C.c_uint64]),
    "gpu_qmoe_layer_desc": (C.c_int, [_vp, _vp, _vp]),
    "gpu_gguf_open": (_vp, [C.c_char_p, C.POINTER(C.c_char_p)]),
    "gpu_gguf_close": (None, [_vp]),
    "gpu_gguf_n_tensors": (C.c_int64, [_vp]),
    "gpu_gguf_n_keys": (C.c_int64, [_vp]),
    "gpu_gguf_find_tensor": (C.c_int64, [_vp, C.c_char_p]),
    "gpu_gguf_tensor_info": (C.c_int, [_vp, C.c_int64, _vp]),
    "gpu_gguf_find_key": (C.c_int64, [_vp, C.c_char_p]),
    "gpu_gguf_key": (C.c_char_p, [_vp, C.c_int64, C.POINTER(C.c_int)]),
    "gpu_gguf_get_int": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_int64)]),
    "gpu_gguf_get_float": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_double)]),
    "gpu_gguf_get_str": (C.c_char_p, [_vp, C.c_char_p]),
    "gpu_gguf_get_arr": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_uint64),
                                   C.POINTER(_vp)]),
    "gpu_gguf_get_arr_str": (C.c_char_p, [_vp, C.c_char_p, C.c_uint64]),
    "gpu_gguf_type_bytes": (C.c_uint64, [C.c_int, C.c_uint64]),
    "gpu_gguf_read_tensor": (C.c_int64, [_vp, C.c_int64, _vp, C.c_uint64]),
    "gpu_gguf_upload_tensor": (C.c_int, [_vp, _vp, C.c_int64, _vp, C.c_uint64]),
    "gpu_gguf_upload_f32": (C.c_int, [_vp, _vp, C.c_int64, _vp, C.c_int64]),
    "gpu_gguf_load_moe_layer": (C.c_int, [_vp, _vp, C.c_int, _vp]),
    "gpu_gguf_free_moe_layer": (None, [_vp, _vp]),
    "gpu_moe_prefill": (C.c_int, [_vp, _vp, _vp, C.c_int, _vp, C.c_int]),
    "gpu_moe_prefill_routing": (C.c_int, [_vp, _vp, _vp]),
    "gpu_f32_to_bf16": (C.c_int, [_vp, _vp, _vp, C.c_int64]),
    "gpu_synth_f32": (C.c_int, [_vp, C.c_uint64, C.c_uint64, C.c_float, _vp, C.c_int64]),
    "gpu_synth_quant": (C.c_int, [_vp, C.c_int, C.c_uint64, C.c_uint64, C.c_uint64, C.c_float,
                                  C.c_int64, C.c_int64, C.c_int, _vp, C.c_uint64]),
    "gpu_synth_zipf_bias": (None, [C.c_uint64, C.c_uint64, C.c_int, C.c_double, _vp]),
    "gpu_timer_start": (C.c_int, [_vp]),
    "gpu_timer_stop": (C.c_float, [_vp]),
}


def load_library(path: str = LIB_PATH) -> C.CDLL:
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run __graft_entry__.build() "
                           "(make -C fomoe_amd); there is no CPU fallback")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    return lib


def row_bytes(t: int, k: int) -> int:
    vals, nb = BLOCK[t]
    if k % vals:
        raise ValueError(f"K={k} is not a multiple of the {vals}-value block of type {t}")
    return k // vals * nb


class MoeLayer(C.Structure):
    """gpu_moe_layer_t (include/gpu.h)."""
    _fields_ = [("n_embd", C.c_int), ("inter", C.c_int), ("n_experts", C.c_int), ("k", C.c_int),
                ("gate_type", C.c_int), ("up_type", C.c_int), ("down_type", C.c_int),
                ("gate_size", C.c_uint64), ("up_size", C.c_uint64), ("expert_stride", C.c_uint64),
                ("router", _vp), ("router_bias", _vp), ("experts", _vp), ("shared", _vp),
                ("shared_inter", C.c_int), ("shared_gate_size", C.c_uint64),
                ("shared_up_size", C.c_uint64), ("shared_gate_vec", _vp), ("norm_w", _vp),
                ("eps", C.c_float), ("shared_gate_type", C.c_int), ("shared_up_type", C.c_int),
                ("shared_down_type", C.c_int)]


class QmoeHeader(C.Structure):
    """Expert-store file header (64 bytes; reference include/expert_store.h:17-29)."""
    _fields_ = [("magic", C.c_uint32), ("version", C.c_uint32), ("n_moe_layers", C.c_uint32),
                ("n_experts", C.c_uint32), ("quant_type", C.c_uint32), ("alignment", C.c_uint32),
                ("expert_gate_size", C.c_uint64), ("expert_up_size", C.c_uint64),
                ("expert_down_size", C.c_uint64), ("expert_stride", C.c_uint64),
                ("reserved", C.c_uint8 * 8)]


class QmoeLayerEntry(C.Structure):
    """Per-layer index entry (32 bytes; reference include/expert_store.h:33-39)."""
    _fields_ = [("data_offset", C.c_uint64), ("expert_stride", C.c_uint64), ("down_size", C.c_uint64),
                ("down_type", C.c_uint32), ("pad", C.c_uint32)]


def qmoe_read_index(path: str, lib=None):
    """Header and layer entries of a .qmoe file (host only); raises on a bad file."""
    lib = lib or load_library()
    h = QmoeHeader()
    err = C.c_char_p()
    n = lib.gpu_qmoe_read_index(path.encode(), C.byref(h), None, 0, C.byref(err))
    if n < 0:
        raise RuntimeError(err.value.decode())
    layers = (QmoeLayerEntry * n)()
    lib.gpu_qmoe_read_index(path.encode(), C.byref(h), layers, n, C.byref(err))
    return h, list(layers)


class GgufTensorInfo(C.Structure):
    """gpu_gguf_tensor_t (include/gpu.h)."""
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_uint32), ("type", C.c_int32),
                ("dims", C.c_int64 * 4), ("offset", C.c_uint64), ("size", C.c_uint64),
                ("split", C.c_int32), ("pad", C.c_int32)]


class Gguf:
    """A GGUF model file opened through the library's reader (host only)."""

    def __init__(self, path: str, lib=None):
        self.lib = lib or load_library()
        err = C.c_char_p()
        self.h = self.lib.gpu_gguf_open(path.encode(), C.byref(err))
        if not self.h:
            raise RuntimeError(err.value.decode())

    def close(self):
        if self.h:
            self.lib.gpu_gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def tensors(self):
        out = []
        for i in range(self.lib.gpu_gguf_n_tensors(self.h)):
            t = GgufTensorInfo()
            assert self.lib.gpu_gguf_tensor_info(self.h, i, C.byref(t)) == 0
            out.append({"name": t.name.decode(), "type": t.type, "dims": list(t.dims[:t.n_dims]),
                        "offset": t.offset, "size": t.size, "split": t.split})
        return out

    def find_tensor(self, name: str) -> int:
        return self.lib.gpu_gguf_find_tensor(self.h, name.encode())

    def keys(self):
        out = []
        for i in range(self.lib.gpu_gguf_n_keys(self.h)):
            ty = C.c_int()
            out.append((self.lib.gpu_gguf_key(self.h, i, C.byref(ty)).decode(), ty.value))
        return out

    def get_int(self, key: str):
        v = C.c_int64()
        return v.value if self.lib.gpu_gguf_get_int(self.h, key.encode(), C.byref(v)) == 0 else None

    def get_float(self, key: str):
        v = C.c_double()
        return v.value if self.lib.gpu_gguf_get_float(self.h, key.encode(), C.byref(v)) == 0 else None

    def get_str(self, key: str):
        v = self.lib.gpu_gguf_get_str(self.h, key.encode())
        return None if v is None else v.decode()

    def get_arr(self, key: str):
        ty, n, data = C.c_int(), C.c_uint64(), _vp()
        if self.lib.gpu_gguf_get_arr(self.h, key.encode(), C.byref(ty), C.byref(n), C.byref(data)) != 0:
            return None
        if ty.value == 8:
            return [self.lib.gpu_gguf_get_arr_str(self.h, key.encode(), i).decode() for i in range(n.value)]
        dt = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32,
              6: np.float32, 7: np.int8, 10: np.uint64, 11: np.int64, 12: np.float64}[ty.value]
        if n.value == 0:
            return np.zeros(0, dt)
        buf = (C.c_uint8 * (n.value * np.dtype(dt).itemsize)).from_address(data.value)
        return np.frombuffer(bytes(buf), dt)

    def read_tensor(self, i: int) -> np.ndarray:
        t = GgufTensorInfo()
        if self.lib.gpu_gguf_tensor_info(self.h, i, C.byref(t)) != 0:
            raise IndexError(i)
        out = np.empty(t.size, np.uint8)
        if self.lib.gpu_gguf_read_tensor(self.h, i, out.ctypes.data, out.size) != t.size:
            raise RuntimeError(f"gguf: reading tensor {i} failed")
        return out


class GpuError(RuntimeError):
    pass


class DeviceBuffer:
    """An owned device allocation."""

    def __init__(self, gpu: "Gpu", nbytes: int):
        self.gpu, self.nbytes = gpu, int(nbytes)
        self.ptr = gpu.lib.gpu_alloc(gpu.ctx, self.nbytes)
        if not self.ptr:
            raise GpuError(f"gpu_alloc({nbytes}) failed: {gpu.last_error()}")

    def free(self):
        if self.ptr:
            self.gpu.lib.gpu_dealloc(self.gpu.ctx, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def offset(self, nbytes: int) -> int:
        return self.ptr + int(nbytes)


class Gpu:
    """One device context (gpu_init/gpu_free)."""

    def __init__(self, lib: C.CDLL | None = None):
        self.lib = lib or load_library()
        self.ctx = self.lib.gpu_init()
        if not self.ctx:
            raise GpuError("gpu_init() returned NULL: no HIP device")
        n_cu, hbm, arch = C.c_int(), C.c_uint64(), C.create_string_buffer(64)
        self.lib.gpu_device_info(self.ctx, C.byref(n_cu), C.byref(hbm), arch, 64)
        self.n_cu, self.hbm, self.arch = n_cu.value, hbm.value, arch.value.decode()

    def close(self):
        if self.ctx:
            self.lib.gpu_free(self.ctx)
            self.ctx = None

    def last_error(self) -> str:
        return (self.lib.gpu_last_error(self.ctx) or b"").decode()

    def check(self, rc: int, what: str):
        if rc != 0:
            raise GpuError(f"{what} failed ({rc}): {self.last_error()}")

    # ------------------------------------------------------------ memory
    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def upload(self, arr: np.ndarray) -> DeviceBuffer:
        arr = np.ascontiguousarray(arr)
        buf = DeviceBuffer(self, max(arr.nbytes, 1))
        self.check(self.lib.gpu_upload(self.ctx, buf.ptr, arr.ctypes.data, arr.nbytes), "gpu_upload")
        return buf

    def upload_to(self, dst, arr: np.ndarray):
        """Copy a host array into an existing device buffer (sync)."""
        arr = np.ascontiguousarray(arr)
        p = dst.ptr if isinstance(dst, DeviceBuffer) else dst
        self.check(self.lib.gpu_upload(self.ctx, p, arr.ctypes.data, arr.nbytes), "gpu_upload")

    def download(self, ptr, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype)
        p = ptr.ptr if isinstance(ptr, DeviceBuffer) else ptr
        self.check(self.lib.gpu_download(self.ctx, out.ctypes.data, p, out.nbytes), "gpu_download")
        return out

    def sync(self):
        self.check(self.lib.gpu_sync(self.ctx), "gpu_sync")

    # ------------------------------------------------------------ kernels
    def dequantize(self, t: int, src: DeviceBuffer, n: int) -> np.ndarray:
        out = self.alloc(4 * n)
        self.check(self.lib.gpu_dequantize(self.ctx, t, src.ptr, out.ptr, n), "gpu_dequantize")
        return self.download(out, np.float32, n)

    def matvec(self, t: int, W, x, y, M: int, K: int):
        self.check(self.lib.gpu_matvec_q(self.ctx, t, _p(W), _p(x), _p(y), M, K), "gpu_matvec_q")

    def matvec_batched(self, t: int, W, mat_stride: int, n_mats: int, x, x_stride: int, y,
                       y_stride: int, M: int, K: int):
        self.check(self.lib.gpu_matvec_q_batched(self.ctx, t, _p(W), mat_stride, n_mats, _p(x),
                                                 x_stride, _p(y), y_stride, M, K),
                   "gpu_matvec_q_batched")

    def moe_layer(self, layer: MoeLayer, x, out, flags: int):
        self.check(self.lib.gpu_moe_layer(self.ctx, C.byref(layer), _p(x), _p(out), flags),
                   "gpu_moe_layer")

    def moe_layer_noalloc(self, layer: MoeLayer, x, out, flags: int) -> int:
        """gpu_moe_layer_noalloc; returns its code (0, or -1 for a layer whose
        scratch exceeds the static area)."""
        return self.lib.gpu_moe_layer_noalloc(self.ctx, C.byref(layer), _p(x), _p(out), flags)

    def last_routing(self, k: int):
        ids = np.empty(k, np.int32)
        w = np.empty(k, np.float32)
        sw = C.c_float()
        self.check(self.lib.gpu_moe_last_routing(self.ctx, ids.ctypes.data, w.ctypes.data,
                                                 C.byref(sw)), "gpu_moe_last_routing")
        return ids, w, sw.value

    def router_topk(self, router, bias, x, norm_w, eps, E, H, k, ids, w):
        self.check(self.lib.gpu_router_topk(self.ctx, _p(router), _p(bias), _p(x), _p(norm_w), eps,
                                            E, H, k, _p(ids), _p(w)), "gpu_router_topk")

    def stack_decode(self, layers, x, n_steps: int):
        arr = (MoeLayer * len(layers))(*layers)
        self.check(self.lib.gpu_moe_stack_decode(self.ctx, arr, len(layers), _p(x), n_steps),
                   "gpu_moe_stack_decode")

    def qmoe_upload_layer(self, path: str, layer: int, dst, nbytes: int):
        self.check(self.lib.gpu_qmoe_upload_layer(self.ctx, path.encode(), layer, _p(dst), nbytes),
                   "gpu_qmoe_upload_layer")

    def qmoe_layer_desc(self, hdr: "QmoeHeader", entry: "QmoeLayerEntry", layer: MoeLayer):
        self.check(self.lib.gpu_qmoe_layer_desc(C.byref(hdr), C.byref(entry), C.byref(layer)),
                   "gpu_qmoe_layer_desc")

    def gguf_upload_tensor(self, g: Gguf, i: int, dst, nbytes: int):
        self.check(self.lib.gpu_gguf_upload_tensor(self.ctx, g.h, i, _p(dst), nbytes), "gpu_gguf_upload_tensor")

    def gguf_upload_f32(self, g: Gguf, i: int, dst, n: int):
        self.check(self.lib.gpu_gguf_upload_f32(self.ctx, g.h, i, _p(dst), n), "gpu_gguf_upload_f32")

    def gguf_load_moe_layer(self, g: Gguf, blk: int) -> MoeLayer:
        L = MoeLayer()
        self.check(self.lib.gpu_gguf_load_moe_layer(self.ctx, g.h, blk, C.byref(L)), "gpu_gguf_load_moe_layer")
        return L

    def gguf_free_moe_layer(self, L: MoeLayer):
        self.lib.gpu_gguf_free_moe_layer(self.ctx, C.byref(L))

    def moe_prefill(self, layer: MoeLayer, x_bf16, n_tokens: int, out, flags: int = 0):
        self.check(self.lib.gpu_moe_prefill(self.ctx, C.byref(layer), _p(x_bf16), n_tokens, _p(out),
                                            flags), "gpu_moe_prefill")

    def prefill_routing(self, n_tokens: int, k: int):
        ids = np.empty((n_tokens, k), np.int32)
        w = np.empty((n_tokens, k + 1), np.float32)
        self.check(self.lib.gpu_moe_prefill_routing(self.ctx, ids.ctypes.data, w.ctypes.data),
                   "gpu_moe_prefill_routing")
        return ids, w

    def f32_to_bf16(self, src, dst, n: int):
        self.check(self.lib.gpu_f32_to_bf16(self.ctx, _p(src), _p(dst), n), "gpu_f32_to_bf16")

    def expert_ffn(self, h: np.ndarray, blobs, scores: np.ndarray, H: int, F: int, gate_size: int,
                   up_size: int, stride: int, gt: int, ut: int, dt: int):
        """Reference-ABI gpu_expert_ffn on host buffers; returns (rc, out)."""
        h = np.ascontiguousarray(h, np.float32)
        scores = np.ascontiguousarray(scores, np.float32)
        ptrs = (C.c_void_p * max(len(blobs), 1))(*[b.ctypes.data for b in blobs])
        out = np.zeros(H, np.float32)
        rc = self.lib.gpu_expert_ffn(self.ctx, h.ctypes.data, ptrs, scores.ctypes.data, len(blobs),
                                     H, F, gate_size, up_size, stride, gt, ut, dt, out.ctypes.data)
        return rc, out

    # ------------------------------------------------------------ synthetic data
    def synth_f32(self, seed: int, stream: int, std: float, out, n: int):
        self.check(self.lib.gpu_synth_f32(self.ctx, seed, stream, std, _p(out), n), "gpu_synth_f32")

    def synth_quant(self, t: int, seed: int, stream0: int, step: int, std: float, M: int, K: int,
                    n_mats: int, dst, dst_stride: int):
        self.check(self.lib.gpu_synth_quant(self.ctx, t, seed, stream0, step, std, M, K, n_mats,
                                            _p(dst), dst_stride), "gpu_synth_quant")

    def zipf_bias(self, seed: int, stream: int, n: int, s: float) -> np.ndarray:
        out = np.empty(n, np.float32)
        self.lib.gpu_synth_zipf_bias(seed, stream, n, s, out.ctypes.data)
        return out

    # ------------------------------------------------------------ timing
    def timer_start(self):
        self.check(self.lib.gpu_timer_start(self.ctx), "gpu_timer_start")

    def timer_stop(self) -> float:
        ms = self.lib.gpu_timer_stop(self.ctx)
        if ms < 0:
            raise GpuError("gpu_timer_stop failed")
        return ms


def _p(x):
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)
