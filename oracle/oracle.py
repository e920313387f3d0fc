"""ctypes view of the CPU oracle (oracle/liboracle.so) and of the reference
build (oracle/_ref/libqwref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker, never as the thing measured
or shipped.  The restated functions live in oracle/qw_oracle.c, each citing the
reference file:line it follows.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i = ctypes.c_int
_i64 = ctypes.c_int64
_fl = ctypes.c_float


def build():
    """Compile the oracle (and oracle/_ref when the reference tree exists)."""
    import subprocess
    subprocess.check_call(["make", "-s", "-C", _HERE, "all"])


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        sig = {
            "orc_f32_to_bf16_n": [_f32p, _u16p, _i64],
            "orc_bf16_to_f32_n": [_u16p, _f32p, _i64],
            "orc_f32_to_f16_n": [_f32p, _u16p, _i64],
            "orc_f16_to_f32_n": [_u16p, _f32p, _i64],
            "orc_linear_f32": [_f32p, _f32p, _f32p, _i, _i, _i],
            "orc_linear_f64": [_f32p, _f32p, _f64p, _i, _i, _i],
            "orc_quantize_rowscale": [_f32p, _i8p, _f32p, _i, _i],
            "orc_linear_int8_dequant": [_i8p, _f32p, _f32p, _f32p, _i, _i, _i],
            "orc_linear_int8_f64": [_i8p, _f32p, _f32p, _f64p, _i, _i, _i],
            "orc_rmsnorm": [_f32p, _f32p, _f32p, _i, _i, _fl],
            "orc_rmsnorm_f64": [_f32p, _f32p, _f64p, _i, _i, ctypes.c_double],
            "orc_residual_rmsnorm": [_f32p, _f32p, _f32p, _f32p, _f32p, _i, _i, _fl],
            "orc_mlp": [_f32p, _f32p, _f32p, _f32p, _f32p, _i, _i, _i],
            "orc_mlp_f64": [_f32p, _f32p, _f32p, _f32p, _f64p, _i, _i, _i],
            "orc_mlp_block": [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i, _i, _i, _fl],
            "orc_mlp_block_f64": [_f32p, _f32p, _f32p, _f32p, _f32p, _f64p, _i, _i, _i, ctypes.c_double],
            "orc_split_q_gate": [_f32p, _f32p, _f32p, _i, _i, _i],
            "orc_argmax_first": [_f32p, _i64],
            "orc_lmhead_argmax": [_f32p, _f32p, _i32p, _f32p, _i, _i, _i],
            "orc_lmhead_argmax_bf16": [_u16p, _u16p, _i32p, _f32p, _i, _i, _i],
            "orc_lmhead_argmax_int8": [_i8p, _f32p, _f32p, _i32p, _f32p, _i, _i, _i],
            "orc_fill_normal": [_f32p, _i64, ctypes.c_uint64, _fl, _fl],
            "orc_fill_uniform": [_f32p, _i64, ctypes.c_uint64, _fl, _fl],
            "orc_fill_int8_uniform": [_i8p, _i64, ctypes.c_uint64, _i, _i],
            "orc_silu": [_fl],
            "orc_gdn_step": [_i, _i, _i, _i, _i, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                             _f32p, _f32p, _f32p],
            "orc_mt64_raw": [ctypes.c_uint64, np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS"), _i64],
            "orc_attn_norm_rope": [_f32p, _f32p, _i, _i, _i, _i, _fl, _f32p, _f32p, _i],
            "orc_kv_quant_int8": [_f32p, _i, _i8p, _f32p],
            "orc_attn_token": [_f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i, _f32p],
            "orc_full_attn_seq": [_i, _i, _i, _i, _i, _i, _fl, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i,
                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, _f32p],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = None
        L.orc_argmax_first.restype = ctypes.c_int32
        L.orc_silu.restype = ctypes.c_float
        _LIB = L
    return _LIB


def ref_lib():
    """The reference's own CPU operators (None when oracle/_ref was not built)."""
    global _REF
    if _REF is None:
        path = os.path.join(_HERE, "_ref", "libqwref.so")
        if not os.path.exists(path):
            return None
        R = ctypes.CDLL(path)
        R.ref_linear.argtypes = [_f32p, _f32p, _f32p, _i, _i, _i]
        R.ref_mlp.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _i, _i, _i]
        R.ref_greedy.argtypes = [_f32p, _i]
        R.ref_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _i, _i, _fl]
        for fn in (R.ref_linear, R.ref_mlp, R.ref_greedy, R.ref_rmsnorm):
            fn.restype = ctypes.c_int
        R.ref_mlp_time.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i]
        R.ref_mlp_time.restype = ctypes.c_double
        R.ref_lmhead_time.argtypes = [_f32p, _f32p, _i, _i, _i, ctypes.c_void_p]
        R.ref_lmhead_time.restype = ctypes.c_double
        R.ref_linear_attn.argtypes = [_f32p, _f32p] + [_i] * 6 + [_f32p] * 11
        R.ref_linear_attn.restype = ctypes.c_int
        R.ref_full_attn.argtypes = [_f32p, _f32p] + [_i] * 6 + [_fl, _fl] + [_f32p] * 6
        R.ref_full_attn.restype = ctypes.c_int
        _REF = R
    return _REF


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---- number formats ------------------------------------------------------
def to_bf16(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_n(x.reshape(-1), out.reshape(-1), x.size)
    return out


def from_bf16(h):
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_bf16_to_f32_n(h.reshape(-1), out.reshape(-1), h.size)
    return out


def to_f16(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(x.reshape(-1), out.reshape(-1), x.size)
    return out


def from_f16(h):
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_n(h.reshape(-1), out.reshape(-1), h.size)
    return out


def round_bf16(x):
    return from_bf16(to_bf16(x))


def round_f16(x):
    return from_f16(to_f16(x))


# ---- projections -----------------------------------------------------------
def linear(W, x):
    W = _c(W, np.float32); x = _c(np.atleast_2d(x), np.float32)
    N, K = W.shape; M = x.shape[0]
    y = np.empty((M, N), np.float32)
    lib().orc_linear_f32(W, x, y, M, N, K)
    return y


def linear_f64(W, x):
    W = _c(W, np.float32); x = _c(np.atleast_2d(x), np.float32)
    N, K = W.shape; M = x.shape[0]
    y = np.empty((M, N), np.float64)
    lib().orc_linear_f64(W, x, y, M, N, K)
    return y


def quantize_rowscale(W):
    W = _c(W, np.float32)
    N, K = W.shape
    q = np.empty((N, K), np.int8); s = np.empty(N, np.float32)
    lib().orc_quantize_rowscale(W, q, s, N, K)
    return q, s


def linear_int8(q, s, x):
    q = _c(q, np.int8); s = _c(s, np.float32); x = _c(np.atleast_2d(x), np.float32)
    N, K = q.shape; M = x.shape[0]
    y = np.empty((M, N), np.float32)
    lib().orc_linear_int8_dequant(q, s, x, y, M, N, K)
    return y


def linear_int8_f64(q, s, x):
    q = _c(q, np.int8); s = _c(s, np.float32); x = _c(np.atleast_2d(x), np.float32)
    N, K = q.shape; M = x.shape[0]
    y = np.empty((M, N), np.float64)
    lib().orc_linear_int8_f64(q, s, x, y, M, N, K)
    return y


def rmsnorm(x, w, eps=1e-6):
    x = _c(np.atleast_2d(x), np.float32); w = _c(w, np.float32)
    M, K = x.shape
    y = np.empty_like(x)
    lib().orc_rmsnorm(x, w, y, M, K, eps)
    return y


def rmsnorm_f64(x, w, eps=1e-6):
    x = _c(np.atleast_2d(x), np.float32); w = _c(w, np.float32)
    M, K = x.shape
    y = np.empty((M, K), np.float64)
    lib().orc_rmsnorm_f64(x, w, y, M, K, eps)
    return y


def residual_rmsnorm(res, a, w, eps=1e-6):
    res = _c(np.atleast_2d(res), np.float32); a = _c(np.atleast_2d(a), np.float32)
    w = _c(w, np.float32)
    M, K = res.shape
    ro = np.empty_like(res); no = np.empty_like(res)
    lib().orc_residual_rmsnorm(res, a, w, ro, no, M, K, eps)
    return ro, no


def silu(v):
    return lib().orc_silu(float(v))


def mlp(Wg, Wu, Wd, x):
    Wg, Wu, Wd = (_c(a, np.float32) for a in (Wg, Wu, Wd))
    x = _c(np.atleast_2d(x), np.float32)
    I, H = Wg.shape; M = x.shape[0]
    y = np.empty((M, H), np.float32)
    lib().orc_mlp(Wg, Wu, Wd, x, y, M, H, I)
    return y


def mlp_f64(Wg, Wu, Wd, x):
    Wg, Wu, Wd = (_c(a, np.float32) for a in (Wg, Wu, Wd))
    x = _c(np.atleast_2d(x), np.float32)
    I, H = Wg.shape; M = x.shape[0]
    y = np.empty((M, H), np.float64)
    lib().orc_mlp_f64(Wg, Wu, Wd, x, y, M, H, I)
    return y


def mlp_block(Wg, Wu, Wd, gamma, x, eps=1e-6):
    Wg, Wu, Wd, gamma = (_c(a, np.float32) for a in (Wg, Wu, Wd, gamma))
    x = _c(np.atleast_2d(x), np.float32)
    I, H = Wg.shape; M = x.shape[0]
    y = np.empty((M, H), np.float32)
    lib().orc_mlp_block(Wg, Wu, Wd, gamma, x, y, M, H, I, eps)
    return y


def mlp_block_f64(Wg, Wu, Wd, gamma, x, eps=1e-6):
    Wg, Wu, Wd, gamma = (_c(a, np.float32) for a in (Wg, Wu, Wd, gamma))
    x = _c(np.atleast_2d(x), np.float32)
    I, H = Wg.shape; M = x.shape[0]
    y = np.empty((M, H), np.float64)
    lib().orc_mlp_block_f64(Wg, Wu, Wd, gamma, x, y, M, H, I, eps)
    return y


def split_q_gate(q_raw, heads, head_dim):
    q_raw = _c(np.atleast_2d(q_raw), np.float32)
    M = q_raw.shape[0]
    q = np.empty((M, heads * head_dim), np.float32); g = np.empty_like(q)
    lib().orc_split_q_gate(q_raw, q, g, M, heads, head_dim)
    return q, g


def argmax_first(v):
    v = _c(v, np.float32).reshape(-1)
    return int(lib().orc_argmax_first(v, v.size))


def lmhead_argmax(E, h):
    E = _c(E, np.float32); h = _c(np.atleast_2d(h), np.float32)
    V, K = E.shape; M = h.shape[0]
    ids = np.empty(M, np.int32); mx = np.empty(M, np.float32)
    lib().orc_lmhead_argmax(E, h, ids, mx, M, V, K)
    return ids, mx


def lmhead_argmax_bf16(E_bits, h_bits):
    E_bits = _c(E_bits, np.uint16); h_bits = _c(np.atleast_2d(h_bits), np.uint16)
    V, K = E_bits.shape; M = h_bits.shape[0]
    ids = np.empty(M, np.int32); mx = np.empty(M, np.float32)
    lib().orc_lmhead_argmax_bf16(E_bits, h_bits, ids, mx, M, V, K)
    return ids, mx


def lmhead_argmax_int8(q, s, h):
    q = _c(q, np.int8); s = _c(s, np.float32); h = _c(np.atleast_2d(h), np.float32)
    V, K = q.shape; M = h.shape[0]
    ids = np.empty(M, np.int32); mx = np.empty(M, np.float32)
    lib().orc_lmhead_argmax_int8(q, s, h, ids, mx, M, V, K)
    return ids, mx


# ---- seeded generator ------------------------------------------------------
def normal(shape, seed, mean=0.0, std=1.0):
    out = np.empty(shape, np.float32)
    lib().orc_fill_normal(out.reshape(-1), out.size, seed, mean, std)
    return out


def uniform(shape, seed, lo, hi):
    out = np.empty(shape, np.float32)
    lib().orc_fill_uniform(out.reshape(-1), out.size, seed, lo, hi)
    return out


def int8_uniform(shape, seed, lo=-127, hi=127):
    out = np.empty(shape, np.int8)
    lib().orc_fill_int8_uniform(out.reshape(-1), out.size, seed, lo, hi)
    return out


def mt64_raw(seed, n):
    out = np.empty(n, np.uint64)
    lib().orc_mt64_raw(seed, out, n)
    return out


# ---- Gated-DeltaNet decode step --------------------------------------------
def gdn_step(mixed, a, b, z, conv_w, A_log, dt_bias, norm_w, conv_state, rec_state, nh, kd, vd):
    """One token per sequence through the step between the projections of
    LinearAttention::forward (language_linear_attn.cpp:143-256).  Returns
    (out [B][nh*vd], conv_state, rec_state), the states as new arrays."""
    mixed = _c(np.atleast_2d(mixed), np.float32)
    B = mixed.shape[0]
    K = conv_w.shape[1]
    cs = _c(conv_state, np.float32).copy()
    rs = _c(rec_state, np.float32).copy()
    out = np.empty((B, nh * vd), np.float32)
    lib().orc_gdn_step(B, nh, kd, vd, K, mixed, _c(a, np.float32), _c(b, np.float32), _c(z, np.float32),
                       _c(conv_w, np.float32), _c(A_log, np.float32), _c(dt_bias, np.float32),
                       _c(norm_w, np.float32), cs, rs, out)
    return out, cs, rs


def ref_linear_attn(x, Wqkv, Wa, Wb, Wz, conv_w, A_log, dt_bias, norm_w, Wout, conv_state, rec_state,
                    nh, kd, vd):
    """The reference's own LinearAttention::forward over the T rows of x (one
    sequence); (y [T][H], conv_state, rec_state)."""
    R = ref_lib()
    x = _c(np.atleast_2d(x), np.float32)
    T, H = x.shape
    y = np.empty((T, H), np.float32)
    cs = _c(conv_state, np.float32).copy()
    rs = _c(rec_state, np.float32).copy()
    rc = R.ref_linear_attn(x, y, T, H, nh, kd, vd, conv_w.shape[1], _c(Wqkv, np.float32), _c(Wa, np.float32),
                           _c(Wb, np.float32), _c(Wz, np.float32), _c(conv_w, np.float32), _c(A_log, np.float32),
                           _c(dt_bias, np.float32), _c(norm_w, np.float32), _c(Wout, np.float32), cs, rs)
    if rc != 0:
        raise RuntimeError("reference LinearAttention raised")
    return y, cs, rs


# ---- gated full attention ----------------------------------------------------
def attn_norm_rope(q, k, q_norm_w, k_norm_w, position, nh, nkv, hd, rotary_dim, theta):
    """Per-head RMSNorm (1 + w) and RoPE of one token's q [nh*hd], k [nkv*hd]
    (language_full_attn.cpp:77-108,156-163); returns new arrays."""
    q = _c(q, np.float32).copy()
    k = _c(k, np.float32).copy()
    lib().orc_attn_norm_rope(q, k, nh, nkv, hd, rotary_dim, theta, _c(q_norm_w, np.float32),
                             _c(k_norm_w, np.float32), int(position))
    return q, k


def kv_quant_int8(x):
    """INT8 of one head vector with its scale (full_attention_cuda.cu:130-150)."""
    x = _c(x, np.float32)
    q = np.empty(x.shape[0], np.int8)
    s = np.empty(1, np.float32)
    lib().orc_kv_quant_int8(x, x.shape[0], q, s)
    return q, float(s[0])


def attn_token(q, gate, kc, vc, nh, nkv, hd):
    """One query token over an FP32 cache [len][nkv][hd], then the sigmoid gate
    (language_full_attn.cpp:165-207)."""
    kc = _c(kc, np.float32)
    out = np.empty(nh * hd, np.float32)
    lib().orc_attn_token(_c(q, np.float32), _c(gate, np.float32), kc, _c(vc, np.float32), kc.shape[0], nh, nkv,
                         hd, out)
    return out


def full_attn_seq(q, gate, k, v, q_norm_w, k_norm_w, nh, nkv, hd, rotary_dim=64, theta=1.0e7, pos0=0,
                  cache=None, int8=False, capacity=None):
    """T tokens of one sequence between the projections: q, gate [T][nh*hd],
    k, v [T][nkv*hd] raw projections.  `cache` = (kc, vc, ks, vs) arrays of
    `capacity` tokens, updated in place (created empty when None).  Returns
    (out [T][nh*hd], cache)."""
    q = _c(np.atleast_2d(q), np.float32)
    T = q.shape[0]
    if cache is None:
        cap = capacity or (pos0 + T)
        kd = np.int8 if int8 else np.float32
        cache = (np.zeros((cap, nkv, hd), kd), np.zeros((cap, nkv, hd), kd), np.zeros((cap, nkv), np.float32),
                 np.zeros((cap, nkv), np.float32))
    kc, vc, ks, vs = cache
    assert kc.shape[0] >= pos0 + T
    out = np.empty((T, nh * hd), np.float32)
    lib().orc_full_attn_seq(T, pos0, nh, nkv, hd, rotary_dim, theta, _c(q_norm_w, np.float32),
                            _c(k_norm_w, np.float32), q, _c(gate, np.float32), _c(k, np.float32),
                            _c(v, np.float32), 1 if int8 else 0, kc.ctypes.data, vc.ctypes.data, ks.ctypes.data,
                            vs.ctypes.data, out)
    return out, cache


def ref_full_attn(x, Wq, Wk, Wv, qn, kn, Wo, nh, nkv, qhd, kvhd, theta=1.0e7, partial=0.25):
    """The reference's own FullAttention::forward over the T rows of x, token t
    at position t from an empty cache; y [T][H]."""
    R = ref_lib()
    x = _c(np.atleast_2d(x), np.float32)
    T, H = x.shape
    y = np.empty((T, H), np.float32)
    rc = R.ref_full_attn(x, y, T, H, nh, nkv, qhd, kvhd, theta, partial, _c(Wq, np.float32), _c(Wk, np.float32),
                         _c(Wv, np.float32), _c(qn, np.float32), _c(kn, np.float32), _c(Wo, np.float32))
    if rc != 0:
        raise RuntimeError("reference FullAttention raised")
    return y
