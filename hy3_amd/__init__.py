"""hy3_amd -- MI355X (gfx950) Hy3 MoE FFN block: host-side binding.

The product is libhy3x.so (HIP, C ABI in include/hy3x_moe.h). This module
loads it with ctypes and wraps the layer object. Device memory and streams
are passed as raw pointers (torch is used only as a convenient allocator by
the tests and the benchmark). There is no CPU fallback: if the library is not
built, every entry point raises.

Reference interface mirrored: the MoE block of yuhai-china/hy3's GPU backend,
gpu_ffn_moe (hy3_gpu.cu:706-738) and its upload in hy3_gpu_init
(hy3_gpu.cu:580-595), with the CPU semantics of forward_layer_moe
(hy3.c:1266-1325).
"""
import ctypes
import os

import numpy as np

__all__ = ["lib", "lib_path", "MoELayer", "HY3XError", "D_MODEL", "D_FF", "N_EXPERT",
           "K_MAX", "Q4K_MATRIX_BYTES", "ROUTE_SCALE", "SHARED", "synth_key",
           "synth_normal", "synth_uniform_sym", "synth_zipf_bias"]

D_MODEL = 4096
D_FF = 1536
N_EXPERT = 192
SHARED = 192
K_MAX = 8
Q4K_BLOCK = 144
Q4K_MATRIX_BYTES = 3538944
Q8_0_MATRIX_BYTES = 7077888  # hy3's Q8_0: 36 bytes per 32 weights
ROUTE_SCALE = 2.826
# Tensor kinds of the synthetic-input specification.
T_X, T_NORM, T_ROUTER, T_BIAS, T_GATE, T_UP, T_DOWN = 1, 2, 3, 4, 5, 6, 7

_HERE = os.path.dirname(os.path.abspath(__file__))
# HY3X_LIBRARY names another build of the same library (A/B measurements)
lib_path = os.environ.get("HY3X_LIBRARY") or os.path.join(_HERE, "libhy3x.so")
_lib = None

P = ctypes.c_void_p
I32 = ctypes.c_int
U32 = ctypes.c_uint32
U64 = ctypes.c_uint64
I64 = ctypes.c_int64
F32 = ctypes.c_float

_SIGS = {
    "hy3x_last_error": (ctypes.c_char_p, []),
    "hy3x_set_device": (I32, [I32]),
    "hy3x_layer_create": (I32, [ctypes.POINTER(P), I32]),
    "hy3x_layer_destroy": (I32, [P]),
    "hy3x_layer_create_shared": (I32, [ctypes.POINTER(P), P]),
    "hy3x_layer_set_router": (I32, [P, P, P, P]),
    "hy3x_layer_set_expert_q4k": (I32, [P, I32, P, P, P, I32]),
    "hy3x_layer_expert_ptr": (I32, [P, I32, I32, ctypes.POINTER(P)]),
    "hy3x_layer_set_shared_q8_0": (I32, [P, P, P, P, I32]),
    "hy3x_layer_load_gguf": (I32, [P, ctypes.c_char_p, I32]),
    "hy3x_gguf_check_layer": (I32, [ctypes.c_char_p, I32, ctypes.POINTER(I32)]),
    "hy3x_synth_shared_q8_0": (I32, [P, U64, U32]),
    "hy3x_synth_quantize_q8_0": (I32, [P, P, I64, P]),
    "hy3x_layer_forward": (I32, [P, P, I32, I32, F32, P]),
    "hy3x_layer_forward_residual": (I32, [P, P, P, I32, I32, F32, P]),
    "hy3x_layer_forward_static": (I32, [P, P, I32, I32, F32, P]),
    "hy3x_layer_last_routing": (I32, [P, P, P, P, I64]),
    "hy3x_layer_last_shape": (I32, [P, ctypes.POINTER(I32), ctypes.POINTER(I32)]),
    "hy3x_layer_set_path": (I32, [P, I32]),
    "hy3x_layer_set_rms_scale": (I32, [P, P, I32]),
    "hy3x_layer_last_path": (I32, [P, ctypes.POINTER(ctypes.c_int)]),
    "hy3x_layer_time_stage": (I32, [P, I32, I32, P, ctypes.POINTER(ctypes.c_float)]),
    "hy3x_layers_time_stage": (I32, [ctypes.POINTER(P), I32, I32, I32, P,
                                     ctypes.POINTER(ctypes.c_float)]),
    "hy3x_diag_read_rate": (I32, [P, I64, I64, I32, P, ctypes.POINTER(ctypes.c_float)]),
    "hy3x_layer_set_timing": (I32, [P, I32]),
    "hy3x_layer_set_trace": (I32, [P, I32, P]),
    "hy3x_layer_stats": (I32, [P, ctypes.POINTER(U64), ctypes.POINTER(U64), I32]),
    "hy3x_layer_stage_times": (I32, [P, P, I32, ctypes.POINTER(I32)]),
    "hy3x_synth_layer_experts": (I32, [P, U64, U32]),
    "hy3x_synth_quantize_q4k": (I32, [P, P, I64, P]),
    "hy3x_synth_key": (U64, [U64, U32, U32, U32]),
    "hy3x_synth_normal": (None, [P, I64, U64, U64, F32, F32]),
    "hy3x_synth_uniform_sym": (None, [P, I64, U64, F32]),
    "hy3x_synth_zipf_bias": (None, [P, I32, U64]),
}


class HY3XError(RuntimeError):
    pass


def one_hip_runtime():
    """Load PyTorch's HIP runtime before anything that links libamdhip64.

    torch ships its own libamdhip64 (soname libamdhip64.so.7) and its
    libraries ask for it by file name. Loaded first, it also serves
    libhy3x.so's libamdhip64.so.7 dependency. Loaded after /opt/rocm's copy,
    the process holds two HIP runtimes, and whichever initialises second
    finds no device. Without torch, libhy3x.so uses /opt/rocm's runtime alone.
    """
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def lib():
    """Load libhy3x.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        one_hip_runtime()
        if not os.path.exists(lib_path):
            raise HY3XError(f"{lib_path} is missing: build it with `python -m hy3_amd.build`")
        h = ctypes.CDLL(lib_path)
        for name, (res, args) in _SIGS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def _check(rc):
    if rc != 0:
        raise HY3XError(f"hy3x error {rc}: {lib().hy3x_last_error().decode()}")


def _ptr(a):
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        assert a.flags["C_CONTIGUOUS"]
        return a.ctypes.data
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    return int(a)


def synth_key(seed, layer, kind, index=0):
    return lib().hy3x_synth_key(seed, layer, kind, index)


def synth_normal(n, key, sigma, offset=0.0, first=0):
    out = np.empty(n, np.float32)
    lib().hy3x_synth_normal(out.ctypes.data, n, key, first, sigma, offset)
    return out


def synth_uniform_sym(n, key, a):
    out = np.empty(n, np.float32)
    lib().hy3x_synth_uniform_sym(out.ctypes.data, n, key, a)
    return out


def synth_zipf_bias(n_expert, seed):
    out = np.empty(n_expert, np.float32)
    lib().hy3x_synth_zipf_bias(out.ctypes.data, n_expert, seed)
    return out


def gguf_check_layer(path, layer_index):
    """Validate a hy3 GGUF file's MoE tensors for one layer (no GPU needed);
    returns the shared expert's ggml type (8: hy3 Q8_0, 12: Q4_K)."""
    t = I32()
    _check(lib().hy3x_gguf_check_layer(os.fsencode(path), layer_index, ctypes.byref(t)))
    return t.value


def layers_time_stage(layers, stage, reps, stream=None):
    """Mean µs per launch of one stage's kernels replayed over `layers` in rotation
    (hy3x_layers_time_stage)."""
    arr = (P * len(layers))(*[L._h for L in layers])
    us = ctypes.c_float()
    _check(lib().hy3x_layers_time_stage(arr, len(layers), MoELayer.STAGES.index(stage), reps,
                                        stream, ctypes.byref(us)))
    return us.value


def read_rate_us(pool_ptr, pool_bytes, nbytes, reps=200, stream=None):
    """Mean µs per launch of a plain streaming read of nbytes (hy3x_diag_read_rate)."""
    us = ctypes.c_float()
    _check(lib().hy3x_diag_read_rate(pool_ptr, pool_bytes, nbytes, reps, stream, ctypes.byref(us)))
    return us.value


class MoELayer:
    """One Hy3 MoE FFN layer resident on the current HIP device."""

    def __init__(self, max_tokens, share_scratch_with=None):
        """share_scratch_with: another MoELayer whose forward scratch this layer
        shares (hy3x_layer_create_shared; forwards of the two must not overlap)."""
        h = P()
        if share_scratch_with is not None:
            _check(lib().hy3x_layer_create_shared(ctypes.byref(h), share_scratch_with._h))
            max_tokens = share_scratch_with.max_tokens
        else:
            _check(lib().hy3x_layer_create(ctypes.byref(h), max_tokens))
        self._h = h
        self.max_tokens = max_tokens

    def close(self):
        if getattr(self, "_h", None):
            lib().hy3x_layer_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_router(self, norm_w, router, bias=None):
        norm_w = np.ascontiguousarray(norm_w, np.float32)
        router = np.ascontiguousarray(router, np.float32)
        assert norm_w.size == D_MODEL and router.size == N_EXPERT * D_MODEL
        if bias is not None:
            bias = np.ascontiguousarray(bias, np.float32)
            assert bias.size == N_EXPERT
        _check(lib().hy3x_layer_set_router(self._h, _ptr(norm_w), _ptr(router), _ptr(bias)))

    def set_expert_q4k(self, expert, gate, up, down, on_device=False):
        if not on_device:
            gate, up, down = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
            assert gate.size == up.size == down.size == Q4K_MATRIX_BYTES
        _check(lib().hy3x_layer_set_expert_q4k(self._h, expert, _ptr(gate), _ptr(up), _ptr(down),
                                               1 if on_device else 0))

    def expert_ptr(self, expert, matrix):
        p = P()
        _check(lib().hy3x_layer_expert_ptr(self._h, expert, matrix, ctypes.byref(p)))
        return p.value

    def synth_experts(self, seed, layer_index=0):
        _check(lib().hy3x_synth_layer_experts(self._h, seed, layer_index))

    def set_shared_q8_0(self, gate, up, down, on_device=False):
        """The shared expert in hy3's Q8_0 (36-byte blocks; hy3x_layer_set_shared_q8_0)."""
        if not on_device:
            gate, up, down = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
            assert gate.size == up.size == down.size == Q8_0_MATRIX_BYTES
        _check(lib().hy3x_layer_set_shared_q8_0(self._h, _ptr(gate), _ptr(up), _ptr(down),
                                                1 if on_device else 0))

    def load_gguf(self, path, layer_index):
        """Router, norm, bias and all 193 experts of one layer from a hy3 GGUF file."""
        _check(lib().hy3x_layer_load_gguf(self._h, os.fsencode(path), layer_index))

    def synth_shared_q8_0(self, seed, layer_index=0):
        _check(lib().hy3x_synth_shared_q8_0(self._h, seed, layer_index))

    path = 0  # 0 auto, 1 GEMV, 2 MFMA, 3 MFMA narrow, 4 MFMA wide (hy3x_layer_set_path)

    def set_path(self, path):
        _check(lib().hy3x_layer_set_path(self._h, path))
        self.path = path

    def last_path(self):
        """Expert path of the last forward: 0 decode kernels, 1 GEMV tiles,
        3 / 4 MFMA narrow / wide tiles."""
        v = ctypes.c_int()
        _check(lib().hy3x_layer_last_path(self._h, ctypes.byref(v)))
        return v.value

    def set_rms_scale(self, r=None):
        """Substitute the per-token RMSNorm scale (None: compute it again)."""
        if r is None:
            _check(lib().hy3x_layer_set_rms_scale(self._h, None, 0))
            return
        r = np.ascontiguousarray(r, np.float32).ravel()
        _check(lib().hy3x_layer_set_rms_scale(self._h, r.ctypes.data, r.size))

    STAGES = ("router", "dispatch", "gateup", "down", "combine")

    def set_timing(self, enable):
        _check(lib().hy3x_layer_set_timing(self._h, 1 if enable else 0))

    def time_stage(self, stage, reps, stream=None):
        """Mean µs per launch of one stage's kernels, replayed `reps` times back to
        back after the last forward (hy3x_layer_time_stage)."""
        us = ctypes.c_float()
        _check(lib().hy3x_layer_time_stage(self._h, self.STAGES.index(stage), reps, stream,
                                           ctypes.byref(us)))
        return us.value

    def stage_times(self):
        """Accumulated ms per stage since the last reset, and the forward count."""
        ms = np.zeros(8, np.float32)
        n = I32()
        _check(lib().hy3x_layer_stage_times(self._h, ms.ctypes.data, 8, ctypes.byref(n)))
        return {k: float(ms[i]) for i, k in enumerate(self.STAGES)}, n.value

    def stats(self, reset=True):
        """(forwards, experts touched summed over forwards) since the last reset."""
        f, u = U64(), U64()
        _check(lib().hy3x_layer_stats(self._h, ctypes.byref(f), ctypes.byref(u), 1 if reset else 0))
        return f.value, u.value

    def forward(self, x_dev_ptr, T, K=K_MAX, scale=ROUTE_SCALE, stream=None):
        """In-place MoE block on device memory x[T x 4096] (fp32)."""
        _check(lib().hy3x_layer_forward(self._h, x_dev_ptr, T, K, scale, stream))

    def forward_static(self, x_dev_ptr, T, K=K_MAX, scale=ROUTE_SCALE, stream=None):
        """forward() on the library's static per-GPU scratch: no allocation
        (hy3x_layer_forward_static; T <= 64)."""
        _check(lib().hy3x_layer_forward_static(self._h, x_dev_ptr, T, K, scale, stream))

    def forward_residual(self, x_dev_ptr, attn_dev_ptr, T, K=K_MAX, scale=ROUTE_SCALE,
                         stream=None):
        """x += attn_out, then the MoE block, in one forward (hy3x_layer_forward_residual)."""
        _check(lib().hy3x_layer_forward_residual(self._h, x_dev_ptr, attn_dev_ptr, T, K, scale,
                                                 stream))

    def last_shape(self):
        """(T, K) of the last forward."""
        t, k = I32(), I32()
        _check(lib().hy3x_layer_last_shape(self._h, ctypes.byref(t), ctypes.byref(k)))
        return t.value, k.value

    def last_routing(self, T=None, K=None):
        """ids, wpre, w of the last forward, each [T x K]. T and K, when given, must be
        the last forward's (they are checked; the buffers are sized from the library's
        own record)."""
        t, k = self.last_shape()
        if (T is not None and T != t) or (K is not None and K != k):
            raise HY3XError(f"last forward was T={t}, K={k}, not T={T}, K={K}")
        ids = np.empty((t, k), np.int32)
        wpre = np.empty((t, k), np.float32)
        w = np.empty((t, k), np.float32)
        _check(lib().hy3x_layer_last_routing(self._h, ids.ctypes.data, wpre.ctypes.data,
                                             w.ctypes.data, ids.size))
        return ids, wpre, w
