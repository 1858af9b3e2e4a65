"""ctypes binding of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker / baseline -- never as the product path.

Also binds the reference shims in oracle/_ref/libhy3ref.so when they have been
built (this container only; they compile yuhai-china/hy3's hy3.c and
hy3_convert.c from /root/reference).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libhy3oracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libhy3ref.so")
D, F, E = 4096, 1536, 192
QB = 144
MAT_BYTES = 3538944
Q8B = 36                      # hy3's Q8_0 block: f32 d + 32 int8
Q8_MAT_BYTES = F * D // 32 * Q8B
TYPE_Q8_0, TYPE_Q4_K = 8, 12
T_X, T_NORM, T_ROUTER, T_BIAS, T_GATE, T_UP, T_DOWN = 1, 2, 3, 4, 5, 6, 7

P = ctypes.c_void_p
I32, U32, U64, I64, F32 = ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int64, ctypes.c_float

_SIGS = {
    "hy3o_splitmix64": (U64, [U64]),
    "hy3o_tensor_key": (U64, [U64, U32, U32, U32]),
    "hy3o_normal": (F32, [U64, U64, F32]),
    "hy3o_uniform_sym": (F32, [U64, U64, F32]),
    "hy3o_fill_normal": (None, [P, ctypes.c_size_t, U64, U64, F32, F32]),
    "hy3o_fill_uniform_sym": (None, [P, ctypes.c_size_t, U64, F32]),
    "hy3o_zipf_bias": (None, [P, I32, U64]),
    "hy3o_fp16_to_fp32": (F32, [ctypes.c_uint16]),
    "hy3o_fp32_to_fp16_trunc": (ctypes.c_uint16, [F32]),
    "hy3o_dequant_q4k": (None, [P, P, I64]),
    "hy3o_quantize_q4k": (None, [P, P, I64]),
    "hy3o_gen_q4k_matrix": (None, [P, I32, I32, U64, F32]),
    "hy3o_quantize_q8_0": (None, [P, P, I64]),
    "hy3o_dequant_q8_0": (None, [P, P, I64]),
    "hy3o_gen_q8_0_matrix": (None, [P, I32, I32, U64, F32]),
    "hy3o_mul_mat_q8_0": (None, [P, P, P, I32, I32]),
    "hy3o_dot8": (F32, [P, P, I32]),
    "hy3o_sig_expf": (F32, [F32]),
    "hy3o_sumsq_block": (F32, [P]),
    "hy3o_rms_norm": (None, [P, P, P, I32]),
    "hy3o_route_token": (None, [P, P, P, P, I32, I32, F32, P, P, P, P, P, P, P]),
    "hy3o_route_token_r": (None, [P, P, P, P, I32, I32, F32, F32, P, P, P, P, P, P, P]),
    "hy3o_topk_select": (None, [P, P, P, I32, I32]),
    "hy3o_mul_mat_q4k": (None, [P, P, P, I32, I32]),
    "hy3o_moe_token": (None, [P, P, I32, F32, P, P, P]),
    "hy3o_moe_forward": (None, [P, P, I32, I32, F32, P, P, P]),
    "hy3o_moe_token_f64": (None, [P, P, P, I32, F32, P]),
    "hy3o_num_threads": (I32, []),
    "hy3o_set_num_threads": (None, [I32]),
}

_REF_SIGS = {
    "hy3ref_fp16_to_fp32": (F32, [ctypes.c_uint16]),
    "hy3ref_dequant_q4k": (None, [P, P, I32]),
    "hy3ref_topk_select": (None, [P, P, P, I32, I32]),
    "hy3ref_mul_mat": (None, [P, P, U32, P, I32, I32]),
    "hy3ref_set_threads": (None, [I32]),
    "hy3ref_moe_forward": (I32, [P, I32, I32, P, P, P, I32, P, P, P, P, I32]),
    "hy3ref_moe_forward_t": (I32, [P, I32, I32, P, P, P, I32, P, P, P, P, I32, U32]),
    "hy3ref_convert": (I32, [ctypes.c_char_p, ctypes.c_char_p, I32]),
    "hy3ref_quantize_q4k": (None, [P, P, I32]),
    "hy3ref_fp32_to_fp16": (ctypes.c_uint16, [F32]),
    "hy3ref_rms_r": (F32, [P, I32]),
    "hy3ref_router_scores": (None, [P, P, P, P, I32, P, P, P]),
}

_lib = None
_ref = None


def build():
    subprocess.run(["make", "-s", "-C", HERE, "libhy3oracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(
                os.path.join(HERE, "hy3_oracle.c")):
            build()
        h = ctypes.CDLL(LIB)
        for n, (r, a) in _SIGS.items():
            f = getattr(h, n)
            f.restype, f.argtypes = r, a
        _lib = h
    return _lib


def ref_lib():
    """The reference shims, or None when oracle/_ref has not been built."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB):
        h = ctypes.CDLL(REF_LIB)
        for n, (r, a) in _REF_SIGS.items():
            f = getattr(h, n)
            f.restype, f.argtypes = r, a
        _ref = h
    return _ref


def ptr(a):
    return None if a is None else a.ctypes.data


class Layer(ctypes.Structure):
    _fields_ = [("norm_w", P), ("router", P), ("bias", P), ("gate", P * (E + 1)),
                ("up", P * (E + 1)), ("down", P * (E + 1)), ("shared_type", I32)]


def key(seed, layer, kind, index=0):
    return lib().hy3o_tensor_key(seed, layer, kind, index)


def normal(n, k, sigma, offset=0.0, first=0):
    out = np.empty(n, np.float32)
    lib().hy3o_fill_normal(out.ctypes.data, n, k, first, sigma, offset)
    return out


def uniform_sym(n, k, a):
    out = np.empty(n, np.float32)
    lib().hy3o_fill_uniform_sym(out.ctypes.data, n, k, a)
    return out


def zipf_bias(n, seed):
    out = np.empty(n, np.float32)
    lib().hy3o_zipf_bias(out.ctypes.data, n, seed)
    return out


def quantize(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size // 256 * QB, np.uint8)
    lib().hy3o_quantize_q4k(x.ctypes.data, out.ctypes.data, x.size)
    return out


def dequant(q):
    q = np.ascontiguousarray(q, np.uint8)
    out = np.empty(q.size // QB * 256, np.float32)
    lib().hy3o_dequant_q4k(out.ctypes.data, q.ctypes.data, out.size)
    return out


def gen_matrix(seed, layer, kind, expert):
    rows, cols = (D, F) if kind == T_DOWN else (F, D)
    out = np.empty(MAT_BYTES, np.uint8)
    lib().hy3o_gen_q4k_matrix(out.ctypes.data, rows, cols, key(seed, layer, kind, expert), 0.02)
    return out


def quantize_q8(x):
    """hy3's Q8_0 quantiser (hy3_convert.c:1192-1221) on a flat fp32 array."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size // 32 * Q8B, np.uint8)
    lib().hy3o_quantize_q8_0(x.ctypes.data, out.ctypes.data, x.size)
    return out


def dequant_q8(q):
    q = np.ascontiguousarray(q, np.uint8)
    out = np.empty(q.size // Q8B * 32, np.float32)
    lib().hy3o_dequant_q8_0(out.ctypes.data, q.ctypes.data, out.size)
    return out


def gen_matrix_q8(seed, layer, kind, expert):
    """The same fp32 values as gen_matrix, quantised to hy3's Q8_0."""
    rows, cols = (D, F) if kind == T_DOWN else (F, D)
    out = np.empty(Q8_MAT_BYTES, np.uint8)
    lib().hy3o_gen_q8_0_matrix(out.ctypes.data, rows, cols, key(seed, layer, kind, expert), 0.02)
    return out


class SynthLayer:
    """CPU copy of a synthetic layer; expert matrices are generated lazily
    (or supplied, e.g. copied back from the device)."""

    def __init__(self, weight_seed, layer=0, zipf_seed=None, has_bias=True, shared_q8=False):
        self.seed, self.layer = weight_seed, layer
        self.shared_q8 = shared_q8  # shared expert in hy3's Q8_0 (real checkpoints)
        self.norm_w = normal(D, key(weight_seed, layer, T_NORM), 0.02, 1.0)
        self.router = normal(E * D, key(weight_seed, layer, T_ROUTER), 0.02)
        if zipf_seed is not None:
            self.bias = zipf_bias(E, zipf_seed)
        else:
            self.bias = uniform_sym(E, key(weight_seed, layer, T_BIAS), 0.1)
        self.has_bias = has_bias
        self.experts = {}

    def expert(self, e):
        if e not in self.experts:
            gen = gen_matrix_q8 if (e == E and self.shared_q8) else gen_matrix
            self.experts[e] = tuple(gen(self.seed, self.layer, k, e)
                                    for k in (T_GATE, T_UP, T_DOWN))
        return self.experts[e]

    def struct(self, needed):
        for e in needed:
            self.expert(e)
        s = Layer()
        s.norm_w, s.router = self.norm_w.ctypes.data, self.router.ctypes.data
        s.bias = self.bias.ctypes.data if self.has_bias else None
        for e, (g, u, d) in self.experts.items():
            s.gate[e], s.up[e], s.down[e] = g.ctypes.data, u.ctypes.data, d.ctypes.data
        s.shared_type = TYPE_Q8_0 if self.shared_q8 else TYPE_Q4_K
        return s

    def route(self, x, K=8, scale=2.826, r_override=None):
        """Routing contract for each row of x: ids, wpre, w, plus s/logits/sigmoid/score.
        r_override[t] > 0 replaces the RMSNorm scale of token t (test hook)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, D)
        T = x.shape[0]
        ids = np.zeros((T, K), np.int32)
        wpre = np.zeros((T, K), np.float32)
        w = np.zeros((T, K), np.float32)
        s = np.zeros((T, D), np.float32)
        lg = np.zeros((T, E), np.float32)
        sg = np.zeros((T, E), np.float32)
        sc = np.zeros((T, E), np.float32)
        L = lib()
        for t in range(T):
            r = 0.0 if r_override is None else float(r_override[t])
            L.hy3o_route_token_r(x[t].ctypes.data, self.norm_w.ctypes.data,
                                 self.router.ctypes.data, self.bias.ctypes.data,
                                 1 if self.has_bias else 0, K, scale, r, s[t].ctypes.data,
                                 lg[t].ctypes.data, sg[t].ctypes.data, sc[t].ctypes.data,
                                 ids[t].ctypes.data, wpre[t].ctypes.data, w[t].ctypes.data)
        return dict(ids=ids, wpre=wpre, w=w, s=s, logits=lg, sigmoid=sg, score=sc)

    def forward(self, x, K=8, scale=2.826):
        """The MoE block (reference semantics) for each row of x; returns y, routing."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, D)
        T = x.shape[0]
        r = self.route(x, K, scale)
        st = self.struct(set(np.unique(r["ids"]).tolist()) | {E})
        y = x.copy()
        ids = np.zeros((T, K), np.int32)
        wpre = np.zeros((T, K), np.float32)
        w = np.zeros((T, K), np.float32)
        lib().hy3o_moe_forward(ctypes.byref(st), y.ctypes.data, T, K, scale, ids.ctypes.data,
                               wpre.ctypes.data, w.ctypes.data)
        return y, dict(ids=ids, wpre=wpre, w=w)

    def forward_f64(self, x, ids, K=8, scale=2.826):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, D)
        st = self.struct(set(np.unique(ids).tolist()) | {E})
        out = np.zeros(x.shape, np.float64)
        for t in range(x.shape[0]):
            idt = np.ascontiguousarray(ids[t], np.int32)
            lib().hy3o_moe_token_f64(ctypes.byref(st), x[t].ctypes.data, out[t].ctypes.data, K,
                                     scale, idt.ctypes.data)
        return out

    def ref_forward(self, x, K=8):
        """The compiled reference forward_layer_moe (needs every expert)."""
        R = ref_lib()
        assert R is not None, "oracle/_ref not built"
        for e in range(E + 1):
            self.expert(e)
        x = np.ascontiguousarray(x, np.float32).reshape(-1, D)
        y = x.copy()
        T = x.shape[0]
        scores = np.zeros((T, E), np.float32)
        ptrs = [(P * (E + 1))(*[self.experts[e][m].ctypes.data for e in range(E + 1)])
                for m in range(3)]
        R.hy3ref_moe_forward_t(y.ctypes.data, T, K, self.norm_w.ctypes.data,
                               self.router.ctypes.data, self.bias.ctypes.data,
                               1 if self.has_bias else 0, ptrs[0], ptrs[1], ptrs[2],
                               scores.ctypes.data, 1, TYPE_Q8_0 if self.shared_q8 else TYPE_Q4_K)
        return y, scores


def topk_select(scores, k):
    scores = np.ascontiguousarray(scores, np.float32)
    vals = np.zeros(k, np.float32)
    inds = np.zeros(k, np.int32)
    lib().hy3o_topk_select(vals.ctypes.data, inds.ctypes.data, scores.ctypes.data, scores.size, k)
    return vals, inds


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))
