"""Python binding of the MI355X projection library (libqw_linear.so, C ABI in
include/qw_linear.h).

The library is the product; this module is a thin ctypes layer so tests,
bench.py and Python callers can drive it.  Device memory and streams come from
PyTorch (tensor.data_ptr(), torch.cuda.current_stream().cuda_stream); nothing
here computes on the host.  If the library is not built the import of `lib()`
raises -- there is no fallback path.

Load this file by path (the package directory name contains dots):
    spec = importlib.util.spec_from_file_location("qw", ".../qw.py")
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqw_linear.so")

# enums (include/qw_linear.h)
OK, ERR_INVALID, ERR_NULL, ERR_SHAPE, ERR_DTYPE, ERR_ALIGN, ERR_WORKSPACE, ERR_HIP, ERR_NOMEM, ERR_STATE = range(10)
F32, BF16, F16, I8 = 0, 1, 2, 3
WFMT_F32, WFMT_BF16, WFMT_INT8 = 0, 1, 2
EP_RESIDUAL, EP_NORM_X, EP_SPLIT = 1, 2, 4

# every symbol include/qw_linear.h declares
EXPORTS = [
    "qw_init", "qw_destroy", "qw_workspace_query", "qw_last_error", "qw_status_string",
    "qw_abi_version", "qw_weight_pack", "qw_weight_pack_glu", "qw_weight_pack_device",
    "qw_weight_pack_glu_device", "qw_weight_pack_concat", "qw_weight_pack_concat_device", "qw_weight_wrap_packed",
    "qw_weight_free", "qw_weight_fold_norm", "qw_weight_info", "qw_weight_device_ptrs", "qw_weight_unpack",
    "qw_linear", "qw_mlp_fused", "qw_layer_tail", "qw_mlp_stack", "qw_device_error", "qw_lmhead_argmax", "qw_lmhead_argmax_noalloc", "qw_argmax_rows", "qw_rmsnorm", "qw_residual_rmsnorm",
    "qw_silu_mul", "qw_gdn_decode", "qw_gdn_prefill", "qw_attn_forward", "qw_embedding_gather", "qw_positions_add", "qw_graph_begin", "qw_graph_end", "qw_graph_launch", "qw_graph_destroy",
    "qw_chain_create", "qw_chain_launch", "qw_chain_destroy", "qw_mlp_stack_epoch", "qw_chain_epoch",
]


class AttnParams(ctypes.Structure):
    _fields_ = [
        ("num_heads", ctypes.c_int),
        ("num_kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("rotary_dim", ctypes.c_int),
        ("rope_theta", ctypes.c_float),
        ("q_norm_weight", ctypes.c_void_p),
        ("k_norm_weight", ctypes.c_void_p),
    ]


class KVCache(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("k_scale", ctypes.c_void_p),
        ("v_scale", ctypes.c_void_p),
        ("capacity", ctypes.c_int),
    ]


class GdnParams(ctypes.Structure):
    _fields_ = [
        ("num_heads", ctypes.c_int),
        ("key_dim", ctypes.c_int),
        ("value_dim", ctypes.c_int),
        ("conv_kernel", ctypes.c_int),
        ("conv_weight", ctypes.c_void_p),
        ("A_log", ctypes.c_void_p),
        ("dt_bias", ctypes.c_void_p),
        ("norm_weight", ctypes.c_void_p),
    ]


class Epilogue(ctypes.Structure):
    _fields_ = [
        ("flags", ctypes.c_uint),
        ("residual", ctypes.c_void_p),
        ("residual_dtype", ctypes.c_int),
        ("ld_residual", ctypes.c_int),
        ("gamma", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("split_period", ctypes.c_int),
        ("y2", ctypes.c_void_p),
    ]


class ChainSlot(ctypes.Structure):
    _fields_ = [
        ("len", ctypes.c_int),
        ("init", ctypes.c_void_p),
        ("ld_init", ctypes.c_int),
        ("out", ctypes.c_void_p),
        ("ld_out", ctypes.c_int),
    ]


class ChainOp(ctypes.Structure):
    _fields_ = [
        ("w", ctypes.c_void_p),
        ("in_", ctypes.c_int),
        ("in_offset", ctypes.c_int),
        ("out", ctypes.c_int),
        ("residual", ctypes.c_int),
        ("norm", ctypes.c_int),
        ("gamma", ctypes.c_void_p),
        ("eps", ctypes.c_float),
    ]


class QwError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"qw status {status}: {msg}")
        self.status = status


_LIB = None
_vp, _i, _sz, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_float


def lib():
    """Load libqw_linear.so (raises if it was not built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built: run __graft_entry__.build() first")
    L = ctypes.CDLL(LIB_PATH)
    pp = ctypes.POINTER(ctypes.c_void_p)
    sigs = {
        "qw_init": ([pp, _i, _sz], _i),
        "qw_destroy": ([_vp], _i),
        "qw_workspace_query": ([_i, _i, _i], _sz),
        "qw_last_error": ([_vp], ctypes.c_char_p),
        "qw_status_string": ([_i], ctypes.c_char_p),
        "qw_abi_version": ([], _i),
        "qw_weight_pack": ([_vp, _vp, _i, _i, _i, _i, _vp, pp], _i),
        "qw_weight_pack_glu": ([_vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, pp], _i),
        "qw_weight_pack_device": ([_vp, _vp, _i, _i, _i, _i, _vp, pp], _i),
        "qw_weight_pack_glu_device": ([_vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, pp], _i),
        "qw_weight_pack_concat": ([_vp, _i, _vp, _vp, _i, _i, _i, _vp, pp], _i),
        "qw_weight_pack_concat_device": ([_vp, _i, _vp, _vp, _i, _i, _i, _vp, pp], _i),
        "qw_weight_wrap_packed": ([_vp, _vp, _vp, _i, _i, _i, pp], _i),
        "qw_weight_fold_norm": ([_vp, _vp, _vp, _vp], _i),
        "qw_weight_free": ([_vp], _i),
        "qw_weight_info": ([_vp, _vp, _vp, _vp, _vp, _vp], _i),
        "qw_weight_device_ptrs": ([_vp, _vp, _vp], _i),
        "qw_weight_unpack": ([_vp, _vp, _vp, _vp], _i),
        "qw_linear": ([_vp, _vp, _vp, _i, _i, _i, _vp, _i, _i, ctypes.POINTER(Epilogue), _vp], _i),
        "qw_mlp_fused": ([_vp, _vp, _vp, _vp, _i, _vp, _f, _vp, _i, _vp, _i, _i, _vp], _i),
        "qw_layer_tail": ([_vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _f, _vp, _i, _vp], _i),
        "qw_gdn_decode": ([_vp, ctypes.POINTER(GdnParams), _i, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _i, _i,
                           _vp], _i),
        "qw_embedding_gather": ([_vp, _vp, _i, _i, _i, _vp, _i, _vp, _i, _i, _vp], _i),
        "qw_positions_add": ([_vp, _vp, _i, _i, _vp], _i),
        "qw_attn_forward": ([_vp, ctypes.POINTER(AttnParams), ctypes.POINTER(KVCache), _i, _i, _vp, _i, _vp, _vp,
                             _i, _vp, _vp, _i, _i, _vp, _i, _i, _vp], _i),
        "qw_gdn_prefill": ([_vp, ctypes.POINTER(GdnParams), _i, _i, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _i,
                            _i, _vp], _i),
        "qw_device_error": ([_vp, _vp], _i),
        "qw_lmhead_argmax": ([_vp, _vp, _vp, _i, _i, _vp, _vp, _vp], _i),
        "qw_mlp_stack": ([_vp, _i, _vp, _vp, _vp, _f, _vp, _i, _vp, _i, _vp], _i),
        "qw_lmhead_argmax_noalloc": ([_vp, _vp, _i, _i, _i, _vp, _i, _i, _vp, _vp, _vp], _i),
        "qw_argmax_rows": ([_vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp], _i),
        "qw_rmsnorm": ([_vp, _vp, _i, _vp, _f, _vp, _i, _i, _i, _vp], _i),
        "qw_residual_rmsnorm": ([_vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _f, _i, _i, _vp], _i),
        "qw_silu_mul": ([_vp, _vp, _vp, _vp, _i, ctypes.c_int64, _vp], _i),
        "qw_graph_begin": ([_vp, _vp], _i),
        "qw_graph_end": ([_vp, _vp, pp], _i),
        "qw_graph_launch": ([_vp, _vp], _i),
        "qw_graph_destroy": ([_vp], _i),
        "qw_chain_create": ([_vp, _i, _i, _i, ctypes.POINTER(ChainSlot), _i, ctypes.POINTER(ChainOp), pp], _i),
        "qw_chain_launch": ([_vp, _vp], _i),
        "qw_chain_destroy": ([_vp], _i),
        "qw_mlp_stack_epoch": ([_vp, _vp, _vp], _i),
        "qw_chain_epoch": ([_vp, _vp, _vp], _i),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _LIB = L
    return L


def _np_dtype_code(a):
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.int8:
        return I8
    raise TypeError(f"unsupported host dtype {a.dtype}; pass float32, int8, or (bits, code)")


def _torch_code(t):
    import torch
    return {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}[t.dtype]


def _stream(stream):
    if stream is None:
        import torch
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if hasattr(stream, "cuda_stream"):
        return ctypes.c_void_p(stream.cuda_stream)
    return ctypes.c_void_p(stream)


class Context:
    """qw_ctx: one per stream; owns the workspace arena."""

    def __init__(self, device=0, workspace_bytes=0):
        self._h = ctypes.c_void_p()
        st = lib().qw_init(ctypes.byref(self._h), device, workspace_bytes)
        if st != OK:
            raise QwError(st, lib().qw_status_string(st).decode())

    @property
    def handle(self):
        return self._h

    def check(self, st):
        if st != OK:
            raise QwError(st, lib().qw_last_error(self._h).decode())

    def device_error(self):
        """Read (and clear) the device error flag (synchronizes)."""
        v = ctypes.c_int()
        self.check(lib().qw_device_error(self._h, ctypes.byref(v)))
        return v.value

    def stack_epoch(self, set_to=None):
        """Test hook: the persistent MLP stack's launch epoch (returned before
        an optional set; synchronizes)."""
        v = ctypes.c_uint()
        st = ctypes.byref(ctypes.c_uint(set_to)) if set_to is not None else None
        self.check(lib().qw_mlp_stack_epoch(self._h, st, ctypes.byref(v)))
        return v.value

    def close(self):
        if self._h:
            lib().qw_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Weight:
    """qw_weight: packed device weight owned by the library."""

    def __init__(self, ctx, handle):
        self.ctx = ctx
        self._h = handle
        N, K, fmt, glu, nbytes = _i(), _i(), _i(), _i(), _sz()
        lib().qw_weight_info(handle, ctypes.byref(N), ctypes.byref(K), ctypes.byref(fmt),
                             ctypes.byref(glu), ctypes.byref(nbytes))
        self.N, self.K, self.fmt, self.glu, self.nbytes = N.value, K.value, fmt.value, glu.value, nbytes.value

    @property
    def handle(self):
        return self._h

    @staticmethod
    def _src(w, src_code):
        if src_code is None:
            w = np.ascontiguousarray(w)
            src_code = _np_dtype_code(w)
        else:
            w = np.ascontiguousarray(w)
        return w, src_code

    @classmethod
    def pack(cls, ctx, w, fmt, scales=None, src_code=None):
        """w: host W[N][K] float32 / int8 (with scales) / uint16 bits + src_code (BF16 or F16)."""
        w, src = cls._src(w, src_code)
        N, K = w.shape
        sc = None if scales is None else np.ascontiguousarray(scales, dtype=np.float32)
        h = ctypes.c_void_p()
        ctx.check(lib().qw_weight_pack(ctx.handle, w.ctypes.data, src, fmt, N, K,
                                       None if sc is None else sc.ctypes.data, ctypes.byref(h)))
        return cls(ctx, h)

    @classmethod
    def pack_glu(cls, ctx, gate, up, fmt, gate_scales=None, up_scales=None, src_code=None):
        gate, src = cls._src(gate, src_code)
        up, _ = cls._src(up, src_code)
        N, K = gate.shape
        gs = None if gate_scales is None else np.ascontiguousarray(gate_scales, dtype=np.float32)
        us = None if up_scales is None else np.ascontiguousarray(up_scales, dtype=np.float32)
        h = ctypes.c_void_p()
        ctx.check(lib().qw_weight_pack_glu(ctx.handle, gate.ctypes.data, up.ctypes.data, src, fmt, N, K,
                                           None if gs is None else gs.ctypes.data,
                                           None if us is None else us.ctypes.data, ctypes.byref(h)))
        return cls(ctx, h)

    @classmethod
    def pack_device(cls, ctx, w, fmt, scales=None):
        """w: torch device tensor W[N][K] (float32/bfloat16/float16, or int8 with
        device float32 scales)."""
        import torch
        code = I8 if w.dtype == torch.int8 else _torch_code(w)
        N, K = w.shape
        h = ctypes.c_void_p()
        ctx.check(lib().qw_weight_pack_device(ctx.handle, w.data_ptr(), code, fmt, N, K,
                                              None if scales is None else scales.data_ptr(), ctypes.byref(h)))
        return cls(ctx, h)

    @classmethod
    def pack_glu_device(cls, ctx, gate, up, fmt, gate_scales=None, up_scales=None):
        import torch
        code = I8 if gate.dtype == torch.int8 else _torch_code(gate)
        N, K = gate.shape
        h = ctypes.c_void_p()
        ctx.check(lib().qw_weight_pack_glu_device(
            ctx.handle, gate.data_ptr(), up.data_ptr(), code, fmt, N, K,
            None if gate_scales is None else gate_scales.data_ptr(),
            None if up_scales is None else up_scales.data_ptr(), ctypes.byref(h)))
        return cls(ctx, h)

    @classmethod
    def pack_concat(cls, ctx, parts, fmt, scales=None, src_code=None):
        """Stack host matrices W_i[N_i][K] (same dtype) into one weight."""
        arrs, src = [], None
        for w in parts:
            w, src = cls._src(w, src_code)
            arrs.append(w)
        K = arrs[0].shape[1]
        ptrs = (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
        Ns = (ctypes.c_int * len(arrs))(*[a.shape[0] for a in arrs])
        scs = None
        if scales is not None:
            keep = [np.ascontiguousarray(v, dtype=np.float32) for v in scales]
            scs = (ctypes.c_void_p * len(keep))(*[v.ctypes.data for v in keep])
        h = ctypes.c_void_p()
        ctx.check(lib().qw_weight_pack_concat(ctx.handle, len(arrs), ptrs, Ns, src, fmt, K, scs, ctypes.byref(h)))
        return cls(ctx, h)

    @classmethod
    def pack_concat_device(cls, ctx, parts, fmt, scales=None):
        """Stack torch device matrices W_i[N_i][K] (scales: device float32 per part, INT8)."""
        import torch
        code = I8 if parts[0].dtype == torch.int8 else _torch_code(parts[0])
        K = parts[0].shape[1]
        ptrs = (ctypes.c_void_p * len(parts))(*[p.data_ptr() for p in parts])
        Ns = (ctypes.c_int * len(parts))(*[p.shape[0] for p in parts])
        scs = None if scales is None else (ctypes.c_void_p * len(scales))(*[v.data_ptr() for v in scales])
        h = ctypes.c_void_p()
        ctx.check(lib().qw_weight_pack_concat_device(ctx.handle, len(parts), ptrs, Ns, code, fmt, K, scs,
                                                     ctypes.byref(h)))
        return cls(ctx, h)

    def fold_norm(self, gamma, stream=None):
        """Multiply (1 + gamma[k]) into the columns (BF16/F32 weights); use the
        weight with gamma=None afterwards (the norm is then rms-only)."""
        self.ctx.check(lib().qw_weight_fold_norm(self.ctx.handle, self._h, _ptr(gamma), _stream(stream)))
        self.norm_folded = True
        return self

    def unpack(self):
        """Stored values as (W rows [parts*N][K] in stored dtype, scales or None)."""
        parts = 2 if self.glu else 1
        dt = {WFMT_F32: np.float32, WFMT_BF16: np.uint16, WFMT_INT8: np.int8}[self.fmt]
        out = np.empty((parts * self.N, self.K), dt)
        sc = np.empty(parts * self.N, np.float32) if self.fmt == WFMT_INT8 else None
        self.ctx.check(lib().qw_weight_unpack(self.ctx.handle, self._h, out.ctypes.data,
                                              None if sc is None else sc.ctypes.data))
        return out, sc

    def device_ptrs(self):
        p, s = ctypes.c_void_p(), ctypes.c_void_p()
        lib().qw_weight_device_ptrs(self._h, ctypes.byref(p), ctypes.byref(s))
        return p.value, s.value

    def free(self):
        if self._h:
            lib().qw_weight_free(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def linear(ctx, W, x, y, residual=None, gamma=None, eps=1e-6, y2=None, split_period=0,
           ldx=0, ldy=0, stream=None, norm=False):
    """y = W.x (+ epilogue) on torch device tensors x [M][>=K], y [M][>=N].
    norm=True without gamma: RMSNorm of x for a weight with a folded norm."""
    ep = Epilogue()
    use_ep = False
    if residual is not None:
        ep.flags |= EP_RESIDUAL
        ep.residual = residual.data_ptr()
        ep.residual_dtype = _torch_code(residual)
        ep.ld_residual = residual.stride(0) if residual.dim() == 2 else 0
        use_ep = True
    if gamma is not None or norm:
        ep.flags |= EP_NORM_X
        ep.gamma = gamma.data_ptr() if gamma is not None else None
        ep.eps = eps
        use_ep = True
    if y2 is not None:
        ep.flags |= EP_SPLIT
        ep.y2 = y2.data_ptr()
        ep.split_period = split_period
        use_ep = True
    M = x.shape[0] if x.dim() == 2 else 1
    ldx = ldx or (x.stride(0) if x.dim() == 2 else 0)
    ldy = ldy or (y.stride(0) if y.dim() == 2 else 0)
    ctx.check(lib().qw_linear(ctx.handle, W.handle, _ptr(x), _torch_code(x), ldx, M, _ptr(y),
                              _torch_code(y), ldy, ctypes.byref(ep) if use_ep else None, _stream(stream)))


def mlp_fused(ctx, gateup, down, x, y, gamma=None, eps=1e-6, residual=None, stream=None):
    M = x.shape[0] if x.dim() == 2 else 1
    ctx.check(lib().qw_mlp_fused(ctx.handle, gateup.handle, down.handle, _ptr(x), _torch_code(x),
                                 _ptr(gamma), eps, _ptr(residual),
                                 _torch_code(residual) if residual is not None else F32,
                                 _ptr(y), _torch_code(y), M, _stream(stream)))


def layer_tail(ctx, w_out, core, gateup, down, x, gamma=None, eps=1e-6, stream=None):
    """qw_layer_tail: x += w_out.core, then x += MLP(RMSNorm(x) (1 + gamma)), on
    the FP32 residual stream x [M][H] in place; core [M][>=K_out] BF16."""
    import torch
    M = x.shape[0] if x.dim() == 2 else 1
    if x.dtype != torch.float32:
        raise TypeError("layer_tail: x must be float32")
    ldc = core.stride(0) if core.dim() == 2 else 0
    ctx.check(lib().qw_layer_tail(ctx.handle, w_out.handle, _ptr(core), _torch_code(core), ldc, gateup.handle,
                                  down.handle, _ptr(gamma), eps, _ptr(x), M, _stream(stream)))


def mlp_stack(ctx, gateups, downs, x, y, gammas=None, eps=1e-6, stream=None):
    """L consecutive MLP blocks (qw_mlp_stack): x [M][1024] -> y, y may be x.
    gammas: L device float tensors, or None when the weights carry the norm."""
    L = len(gateups)
    M = x.shape[0] if x.dim() == 2 else 1
    gu = (ctypes.c_void_p * L)(*[w.handle.value for w in gateups])
    dn = (ctypes.c_void_p * L)(*[w.handle.value for w in downs])
    gm = None if gammas is None else (ctypes.c_void_p * L)(*[g.data_ptr() for g in gammas])
    ctx.check(lib().qw_mlp_stack(ctx.handle, L, gu, dn, gm, eps, _ptr(x), _torch_code(x), _ptr(y), M,
                                 _stream(stream)))


def lmhead_argmax(ctx, E, h, ids, max_logit=None, stream=None):
    M = h.shape[0] if h.dim() == 2 else 1
    ctx.check(lib().qw_lmhead_argmax(ctx.handle, E.handle, _ptr(h), _torch_code(h), M, _ptr(ids),
                                     _ptr(max_logit), _stream(stream)))


def lmhead_argmax_noalloc(E, h, ids, max_logit=None, stream=None):
    """qw_lmhead_argmax_noalloc over the packed device data of Weight E (no
    context: the argmax keys live in the library's per-device array)."""
    M = h.shape[0] if h.dim() == 2 else 1
    packed, scales = E.device_ptrs()
    st = lib().qw_lmhead_argmax_noalloc(packed, scales, E.fmt, E.N, E.K, _ptr(h), _torch_code(h), M, _ptr(ids),
                                        _ptr(max_logit), _stream(stream))
    if st != OK:
        raise QwError(st, lib().qw_status_string(st).decode())


def argmax_rows(ctx, logits, ids, max_logit=None, stream=None):
    """Greedy argmax of each row of logits [M][V] (lowest index on ties)."""
    M, V = logits.shape
    ctx.check(lib().qw_argmax_rows(ctx.handle, _ptr(logits), _torch_code(logits), M, V, logits.stride(0),
                                   _ptr(ids), _ptr(max_logit), _stream(stream)))


def rmsnorm(ctx, x, gamma, y, eps=1e-6, stream=None):
    M, K = x.shape
    ctx.check(lib().qw_rmsnorm(ctx.handle, _ptr(x), _torch_code(x), _ptr(gamma), eps, _ptr(y),
                               _torch_code(y), M, K, _stream(stream)))


def residual_rmsnorm(ctx, residual_in, a, residual_out, normed, gamma, eps=1e-6, stream=None):
    M, K = residual_in.shape
    ctx.check(lib().qw_residual_rmsnorm(ctx.handle, _ptr(residual_in), _ptr(a), _torch_code(residual_in),
                                        _ptr(residual_out), _ptr(normed), _torch_code(normed),
                                        _ptr(gamma), eps, M, K, _stream(stream)))


def silu_mul(ctx, g, u, h, stream=None):
    ctx.check(lib().qw_silu_mul(ctx.handle, _ptr(g), _ptr(u), _ptr(h), _torch_code(g), g.numel(),
                                _stream(stream)))


class Chain:
    """A chain of dependent projections run as one persistent launch
    (qw_chain_create / qw_chain_launch).

    slots: list of dicts {len, init (tensor [M][>=len] or None), out (tensor or None)};
    ops: list of dicts {w: Weight, in, out, in_offset=0, residual=False,
    gamma=None (tensor), norm=False, eps=1e-6}.  The tensors must stay alive
    as long as the chain (their device addresses are baked into the plan)."""

    def __init__(self, ctx, act_code, M, slots, ops):
        self.ctx, self._keep = ctx, []
        ss = (ChainSlot * len(slots))()
        for i, sl in enumerate(slots):
            ss[i].len = sl["len"]
            for key, ldk in (("init", "ld_init"), ("out", "ld_out")):
                t = sl.get(key)
                if t is not None:
                    setattr(ss[i], key, t.data_ptr())
                    setattr(ss[i], ldk, t.stride(0) if t.dim() == 2 else 0)
                    self._keep.append(t)
        oo = (ChainOp * len(ops))()
        for i, op in enumerate(ops):
            oo[i].w = op["w"].handle.value
            oo[i].in_ = op["in"]
            oo[i].in_offset = op.get("in_offset", 0)
            oo[i].out = op["out"]
            oo[i].residual = 1 if op.get("residual") else 0
            g = op.get("gamma")
            oo[i].norm = 1 if (op.get("norm") or g is not None) else 0
            if g is not None:
                oo[i].gamma = g.data_ptr()
                self._keep.append(g)
            oo[i].eps = op.get("eps", 1e-6)
            self._keep.append(op["w"])
        self._h = ctypes.c_void_p()
        ctx.check(lib().qw_chain_create(ctx.handle, act_code, M, len(slots), ss, len(ops), oo, ctypes.byref(self._h)))

    def launch(self, stream=None):
        self.ctx.check(lib().qw_chain_launch(self._h, _stream(stream)))

    def epoch(self, set_to=None):
        """Test hook: the chain's launch epoch (returned before an optional
        set; synchronizes)."""
        v = ctypes.c_uint()
        st = ctypes.byref(ctypes.c_uint(set_to)) if set_to is not None else None
        self.ctx.check(lib().qw_chain_epoch(self._h, st, ctypes.byref(v)))
        return v.value

    def close(self):
        if self._h:
            lib().qw_chain_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Graph:
    """Capture qw_* calls on a stream and replay them."""

    def __init__(self, ctx, stream):
        self.ctx, self.stream, self._h = ctx, stream, ctypes.c_void_p()

    def __enter__(self):
        self.ctx.check(lib().qw_graph_begin(self.ctx.handle, _stream(self.stream)))
        return self

    def __exit__(self, *exc):
        self.ctx.check(lib().qw_graph_end(self.ctx.handle, _stream(self.stream), ctypes.byref(self._h)))
        return False

    def launch(self, stream=None):
        st = lib().qw_graph_launch(self._h, _stream(stream if stream is not None else self.stream))
        if st != OK:
            raise QwError(st, "graph launch failed")

    def __del__(self):
        try:
            if self._h:
                lib().qw_graph_destroy(self._h)
        except Exception:
            pass


def gdn_decode(ctx, conv_weight, A_log, dt_bias, norm_weight, mixed, z, a, b, conv_state, recurrent_state, out,
               num_heads, key_dim=128, value_dim=128, ld_in=0, ld_out=0, stream=None):
    """Gated-DeltaNet decode step for the rows (sequences) of mixed/z/a/b
    (views into one projection output share its row stride); the FP32
    states are updated in place; out [B][>= num_heads*value_dim]."""
    p = GdnParams(num_heads, key_dim, value_dim, conv_weight.shape[1], conv_weight.data_ptr(), A_log.data_ptr(),
                  dt_bias.data_ptr(), norm_weight.data_ptr())
    B = mixed.shape[0]
    ld_in = ld_in or mixed.stride(0)
    ld_out = ld_out or out.stride(0)
    ctx.check(lib().qw_gdn_decode(ctx.handle, ctypes.byref(p), B, _ptr(mixed), _ptr(z), _ptr(a), _ptr(b),
                                  _torch_code(mixed), ld_in, _ptr(conv_state), _ptr(recurrent_state), _ptr(out),
                                  _torch_code(out), ld_out, _stream(stream)))


def gdn_prefill(ctx, conv_weight, A_log, dt_bias, norm_weight, mixed, z, a, b, conv_state, recurrent_state, out,
                num_heads, tokens, key_dim=128, value_dim=128, ld_in=0, ld_out=0, stream=None):
    """Gated-DeltaNet step over `tokens` consecutive tokens of each sequence:
    row s*tokens + t of mixed/z/a/b/out is token t of sequence s; the FP32
    states (one per sequence) carry across the tokens and are updated in
    place."""
    p = GdnParams(num_heads, key_dim, value_dim, conv_weight.shape[1], conv_weight.data_ptr(), A_log.data_ptr(),
                  dt_bias.data_ptr(), norm_weight.data_ptr())
    rows = mixed.shape[0]
    if tokens < 1 or rows % tokens:
        raise QwError(ERR_SHAPE, f"{rows} rows are not a whole number of {tokens}-token sequences")
    ld_in = ld_in or mixed.stride(0)
    ld_out = ld_out or out.stride(0)
    ctx.check(lib().qw_gdn_prefill(ctx.handle, ctypes.byref(p), rows // tokens, tokens, _ptr(mixed), _ptr(z),
                                   _ptr(a), _ptr(b), _torch_code(mixed), ld_in, _ptr(conv_state),
                                   _ptr(recurrent_state), _ptr(out), _torch_code(out), ld_out, _stream(stream)))


def kv_cache(sequences, capacity, num_kv_heads=2, head_dim=256, int8=True, device="cuda"):
    """Zeroed device KV cache of one layer: (k, v, k_scale, v_scale) tensors in
    the qw_kv_cache layout [sequences][capacity][num_kv_heads][head_dim]."""
    import torch
    dt = torch.int8 if int8 else torch.float32
    shape = (sequences, capacity, num_kv_heads, head_dim)
    return (torch.zeros(shape, dtype=dt, device=device), torch.zeros(shape, dtype=dt, device=device),
            torch.zeros(shape[:3], dtype=torch.float32, device=device),
            torch.zeros(shape[:3], dtype=torch.float32, device=device))


def attn_forward(ctx, q_norm_weight, k_norm_weight, cache, positions, q, gate, k, v, out, num_heads=8,
                 num_kv_heads=2, head_dim=256, rotary_dim=64, rope_theta=1.0e7, tokens=1, q_head_stride=0,
                 ld_in=0, ld_out=0, max_len=0, stream=None):
    """Gated full attention between the projections for rows = batch*tokens
    (row b*tokens + t is token t of sequence b at position positions[b] + t);
    q/gate/k/v are views into the projection output(s) sharing one row stride;
    `cache` is kv_cache(...)'s tuple, updated in place."""
    kc, vc, ks, vs = cache
    p = AttnParams(num_heads, num_kv_heads, head_dim, rotary_dim, rope_theta, q_norm_weight.data_ptr(),
                   k_norm_weight.data_ptr())
    int8 = kc.element_size() == 1
    c = KVCache(I8 if int8 else F32, kc.data_ptr(), vc.data_ptr(), ks.data_ptr() if int8 else None,
                vs.data_ptr() if int8 else None, kc.shape[1])
    rows = q.shape[0]
    if tokens < 1 or rows % tokens:
        raise QwError(ERR_SHAPE, f"{rows} rows are not a whole number of {tokens}-token sequences")
    ld_in = ld_in or q.stride(0)
    ld_out = ld_out or out.stride(0)
    q_head_stride = q_head_stride or head_dim
    ctx.check(lib().qw_attn_forward(ctx.handle, ctypes.byref(p), ctypes.byref(c), rows // tokens, tokens,
                                    _ptr(positions), max_len, _ptr(q), _ptr(gate), q_head_stride, _ptr(k), _ptr(v),
                                    _torch_code(q), ld_in, _ptr(out), _torch_code(out), ld_out, _stream(stream)))


def embedding_gather(ctx, table, ids, out, ld_out=0, stream=None):
    """out[m] = table[ids[m]] (table [vocab][hidden] F32 or BF16; ids int32)."""
    ctx.check(lib().qw_embedding_gather(ctx.handle, _ptr(table), _torch_code(table), table.shape[0], table.shape[1],
                                        _ptr(ids), ids.shape[0], _ptr(out), _torch_code(out),
                                        ld_out or out.stride(0), _stream(stream)))


def positions_add(ctx, positions, delta=1, stream=None):
    ctx.check(lib().qw_positions_add(ctx.handle, _ptr(positions), positions.numel(), delta, _stream(stream)))
