"""Whole-model greedy decode step for Qwen3.5-0.8B on the C ABI (libqw_linear).

One step takes the current token of each of B sequences to the next one,
entirely on the device:

    x    = embedding[ids]                                   qw_embedding_gather
    per layer (the CPU LanguageBackbone order, language_backbone.cpp:54-88):
      x += attn(RMSNorm(x) * (1 + w_in))                    in-projection with the
                                                            norm prologue, core,
                                                            out-projection + residual
           linear layers: qw_gdn_decode (Gated-DeltaNet state per sequence)
           full layers (3, 7, 11, 15, 19, 23; is_linear_layer,
           language_common.hpp:36-44): qw_attn_forward over the KV cache
      x += MLP(RMSNorm(x) * (1 + w_post))                   qw_mlp_fused
    ids  = argmax(E . RMSNorm(x) * (1 + w_final))           qw_rmsnorm + qw_lmhead_argmax
    positions += 1                                          qw_positions_add

No host synchronization and no allocation inside a step, so the step can be
captured once (qw.Graph) and replayed per token.  Weights are random-init
synthetic tensors of the real shapes in the benchmark (no checkpoint is
available); the reference's flat per-layer layout (WEIGHT_FORMAT.md, read by
CudaEngine::set_layer_weights, cuda_engine.cu:244-298) is what `layers`
mirrors by name.
"""

H, I, V_DEFAULT = 1024, 3584, 248320
LNH, KD, VD, CK = 16, 128, 128, 4           # linear attention
CD = LNH * (2 * KD + VD)                    # conv dim 6144
LIN_IN = CD + LNH * VD + 2 * LNH            # stacked [qkv | z | a | b] = 8224
FNH, FNKV, HD = 8, 2, 256                   # full attention
FULL_IN = FNH * 2 * HD + 2 * FNKV * HD      # stacked [q|gate interleaved | k | v] = 5120
NORM_FIRST_MIN_BATCH = 12                   # above this many sequences, RMSNorm once into BF16


def is_linear_layer(i):
    """language_common.hpp:36-44: every fourth layer (3, 7, ...) is full attention."""
    return i % 4 != 3


class DecodeEngine:
    """Device-resident model + per-sequence state for greedy decoding of B sequences.

    layers: list of dicts of torch float32 CUDA tensors named as the reference
    flat layout: in_norm, post_norm, gate, up, down, and for linear layers
    qkv, a, b, z, conv, out, A_log, dt_bias, norm_w; for full layers q, k, v,
    q_norm, k_norm, o.  embed: [vocab][H] (F32 or BF16, the tied lm_head)."""

    def __init__(self, qw, ctx, layers, final_norm, embed, batch, capacity, fmt=None, lm_fmt=None,
                 kv_int8=True, norm_first=None):
        import torch
        self.qw, self.ctx, self.B = qw, ctx, batch
        fmt = qw.WFMT_BF16 if fmt is None else fmt
        lm_fmt = qw.WFMT_BF16 if lm_fmt is None else lm_fmt
        dev = "cuda"
        self.act = torch.float32 if fmt == qw.WFMT_F32 else torch.bfloat16
        # Where the layer input is RMSNorm-ed: inside the projection (its
        # prologue stages the FP32 residual stream per workgroup), or once into
        # a BF16 buffer that the register-direct GEMV reads.  The prologue wins
        # for few sequences (one launch fewer: ~4.4 us each in the step graph);
        # with many, every workgroup re-staging x (M x 4 KB) costs more than
        # the extra launch.  Measured whole-step crossover between 8 and 16
        # sequences (B=8: 1.108 vs 1.206 ms, B=16: 1.487 vs 1.449 ms, B=32:
        # 2.57 vs 1.85 ms).  BF16 weights only: FP32 weights keep FP32 x.
        if norm_first is None:
            norm_first = self.act == torch.bfloat16 and batch > NORM_FIRST_MIN_BATCH
        self.norm_first = bool(norm_first)
        self.layers = []
        for i, L in enumerate(layers):
            P = {"linear": is_linear_layer(i), "in_norm": L["in_norm"], "post_norm": L["post_norm"]}
            P["gateup"] = qw.Weight.pack_glu_device(ctx, L["gate"], L["up"], fmt)
            P["down"] = qw.Weight.pack_device(ctx, L["down"], fmt)
            if P["linear"]:
                P["in"] = qw.Weight.pack_concat_device(ctx, [L["qkv"], L["z"], L["a"], L["b"]], fmt)
                P["out"] = qw.Weight.pack_device(ctx, L["out"], fmt)
                for n in ("conv", "A_log", "dt_bias", "norm_w"):
                    P[n] = L[n].contiguous()
                P["cs"] = torch.zeros(batch, CD, CK - 1, device=dev)
                P["rs"] = torch.zeros(batch, LNH, KD * VD, device=dev)
            else:
                P["in"] = qw.Weight.pack_concat_device(ctx, [L["q"], L["k"], L["v"]], fmt)
                P["out"] = qw.Weight.pack_device(ctx, L["o"], fmt)
                P["q_norm"], P["k_norm"] = L["q_norm"].contiguous(), L["k_norm"].contiguous()
                P["cache"] = qw.kv_cache(batch, capacity, FNKV, HD, int8=kv_int8)
            self.layers.append(P)
        self.final_norm = final_norm
        self.embed = embed
        self.E = qw.Weight.pack_device(ctx, embed.float() if embed.dtype != torch.float32 else embed, lm_fmt)
        self.capacity = capacity
        self.x = torch.zeros(batch, H, device=dev)
        self.xn = torch.zeros(batch, H, device=dev)
        self.xh = torch.zeros(batch, H, device=dev, dtype=torch.bfloat16)  # RMSNorm-ed x (norm_first)
        self.row = torch.zeros(batch, max(LIN_IN, FULL_IN), device=dev)
        self.core = torch.zeros(batch, LNH * VD, device=dev, dtype=self.act)
        self.ids = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(batch, dtype=torch.int32, device=dev)

    def reset(self, ids, positions=None):
        """Start B sequences at token ids (and positions, default 0) with cleared states."""
        import torch
        self.ids.copy_(torch.as_tensor(ids, dtype=torch.int32))
        self.pos.copy_(torch.as_tensor(positions if positions is not None else [0] * self.B, dtype=torch.int32))
        for P in self.layers:
            if P["linear"]:
                P["cs"].zero_()
                P["rs"].zero_()
            else:
                for c in P["cache"]:
                    c.zero_()

    def check(self):
        """Raise if a kernel of the steps since the last check raised the
        context's device error flag (a token outside its KV cache, an
        embedding id outside the vocabulary, or an expired wait of the
        one-launch MLP): their outputs are invalid.  Reads and clears the flag
        (synchronizes the device), so it is never called inside a graph
        capture; after replaying a captured step, call it from the host."""
        flag = self.ctx.device_error()
        if flag:
            raise RuntimeError(f"device error flag {flag}: the last steps' outputs are invalid")

    def prefill(self, ids, stream=None, check=None):
        """T prompt tokens of every sequence in one pass (ids: device int32
        [B][T]), from each sequence's current position -- the batched
        counterpart of step(), as CudaEngine::forward_batch_prefill
        (cuda_engine.cu:354-389) for B sequences.  Every projection sees
        M = B*T rows (the MFMA GEMM from 33 rows on, so the layer inputs are
        RMSNorm-ed once into the weights' activation type), Gated-DeltaNet runs
        its chunked form from 24 tokens on and full attention its query-block
        kernel from 16.  The states and caches advance by T; self.ids receives
        the greedy next token of every sequence and self.pos += T.
        check (default: when no stream is given) reads the device error flag
        afterwards and raises if it was set (see check()); that read
        synchronizes the device (check=False keeps the call asynchronous)."""
        import torch
        qw, ctx = self.qw, self.ctx
        B, T = ids.shape
        if B != self.B:
            raise ValueError(f"prefill: ids has {B} sequences, the engine {self.B}")
        M = B * T
        dev = self.x.device
        X = torch.empty(M, H, device=dev)
        Xn = torch.empty(M, H, device=dev, dtype=self.act)
        row = torch.empty(M, max(LIN_IN, FULL_IN), device=dev)
        core = torch.empty(M, LNH * VD, device=dev, dtype=self.act)
        qw.embedding_gather(ctx, self.embed, ids.reshape(-1).contiguous(), X, stream=stream)
        for P in self.layers:
            qw.rmsnorm(ctx, X, P["in_norm"], Xn, stream=stream)
            if P["linear"]:
                r = row[:, :LIN_IN]
                qw.linear(ctx, P["in"], Xn, r, stream=stream)
                qw.gdn_prefill(ctx, P["conv"], P["A_log"], P["dt_bias"], P["norm_w"], r[:, :CD],
                               r[:, CD:CD + LNH * VD], r[:, CD + LNH * VD:CD + LNH * VD + LNH],
                               r[:, CD + LNH * VD + LNH:], P["cs"], P["rs"], core, LNH, T, ld_in=row.stride(0),
                               stream=stream)
            else:
                r = row[:, :FULL_IN]
                qw.linear(ctx, P["in"], Xn, r, stream=stream)
                qw.attn_forward(ctx, P["q_norm"], P["k_norm"], P["cache"], self.pos, r[:, 0:], r[:, HD:],
                                r[:, FNH * 2 * HD:], r[:, FNH * 2 * HD + FNKV * HD:], core, tokens=T,
                                q_head_stride=2 * HD, ld_in=row.stride(0), max_len=self.capacity, stream=stream)
            qw.linear(ctx, P["out"], core, X, residual=X, stream=stream)
            qw.rmsnorm(ctx, X, P["post_norm"], Xn, stream=stream)
            qw.mlp_fused(ctx, P["gateup"], P["down"], Xn, X, residual=X, stream=stream)
        if stream is None:
            self.x.copy_(X.view(B, T, H)[:, T - 1])
        else:
            with torch.cuda.stream(stream):
                self.x.copy_(X.view(B, T, H)[:, T - 1])
        qw.rmsnorm(ctx, self.x, self.final_norm, self.xn, stream=stream)
        qw.lmhead_argmax(ctx, self.E, self.xn, self.ids, stream=stream)
        qw.positions_add(ctx, self.pos, T, stream=stream)
        if check if check is not None else stream is None:
            self.check()

    def _project_in(self, P, r, stream):
        """The layer's stacked input projection of RMSNorm(x) * (1 + in_norm)."""
        qw, ctx = self.qw, self.ctx
        if self.norm_first:
            qw.rmsnorm(ctx, self.x, P["in_norm"], self.xh, stream=stream)
            qw.linear(ctx, P["in"], self.xh, r, stream=stream)
        else:
            qw.linear(ctx, P["in"], self.x, r, gamma=P["in_norm"], stream=stream)

    def step(self, stream=None, check=None):
        """One greedy token for every sequence: ids <- next ids, positions += 1.
        check (default: when no stream is given, i.e. never while a graph is
        captured on a stream) reads the device error flag afterwards and
        raises if it was set (see check()); that read synchronizes the device,
        so an eager step with the default blocks the host until it is done.
        Pass check=False (or a stream) to keep eager steps asynchronous and
        call check() every N steps instead."""
        qw, ctx, x, row = self.qw, self.ctx, self.x, self.row
        qw.embedding_gather(ctx, self.embed, self.ids, x, stream=stream)
        for P in self.layers:
            if P["linear"]:
                r = row[:, :LIN_IN]
                self._project_in(P, r, stream)
                qw.gdn_decode(ctx, P["conv"], P["A_log"], P["dt_bias"], P["norm_w"], r[:, :CD],
                              r[:, CD:CD + LNH * VD], r[:, CD + LNH * VD:CD + LNH * VD + LNH],
                              r[:, CD + LNH * VD + LNH:], P["cs"], P["rs"], self.core, LNH, ld_in=row.stride(0),
                              stream=stream)
            else:
                r = row[:, :FULL_IN]
                self._project_in(P, r, stream)
                qw.attn_forward(ctx, P["q_norm"], P["k_norm"], P["cache"], self.pos, r[:, 0:], r[:, HD:],
                                r[:, FNH * 2 * HD:], r[:, FNH * 2 * HD + FNKV * HD:], self.core, tokens=1,
                                q_head_stride=2 * HD, ld_in=row.stride(0), max_len=self.capacity, stream=stream)
            if self.norm_first:
                qw.linear(ctx, P["out"], self.core, x, residual=x, stream=stream)
                qw.rmsnorm(ctx, x, P["post_norm"], self.xh, stream=stream)
                qw.mlp_fused(ctx, P["gateup"], P["down"], self.xh, x, residual=x, stream=stream)
            else:
                # out-projection + residual, post-norm MLP + residual: one launch at decode sizes
                qw.layer_tail(ctx, P["out"], self.core, P["gateup"], P["down"], x, gamma=P["post_norm"],
                              stream=stream)
        qw.rmsnorm(ctx, x, self.final_norm, self.xn, stream=stream)
        qw.lmhead_argmax(ctx, self.E, self.xn, self.ids, stream=stream)
        qw.positions_add(ctx, self.pos, 1, stream=stream)
        if check if check is not None else stream is None:
            self.check()


# ---------------------------------------------------------------------------
# Weight loaders.  The reference carries three layouts of the same tensors,
# all raw little-endian FP32:
#   (A) a directory tree, one file per tensor, matrices [out][in] as the CPU
#       operators consume them: weights/language/embed_tokens.bin,
#       weights/language_backbone/layer_N/{input_layernorm, post_layernorm,
#       mlp_gate, mlp_up, mlp_down, linear_qkv, linear_a, linear_b, linear_z,
#       linear_conv1d, linear_A_log, linear_dt_bias, linear_norm, linear_out,
#       full_q, full_k, full_v, full_q_norm, full_k_norm, full_o}.bin and
#       weights/language_backbone/final_norm.bin
#       (tests/integration/e2e_validate.cpp:37-84,126);
#   (B) one flat vector per layer as CudaEngine::set_layer_weights slices it
#       (cuda_engine.cu:244-298): the common prefix (norms, MLP), then the
#       whole linear-attention section, then the whole full-attention section,
#       matrices [out][in];
#   (C) the files of scripts/export_real_weights.py: weights/layer_XX.bin with
#       the common prefix and only the layer type's own section, every matrix
#       transposed to [in][out] by its transpose_if_needed (:43-48), plus
#       norm.bin and embedding.bin.
# All three load into the `layers` dicts DecodeEngine takes ([out][in]).

_COMMON = [("in_norm", (H,)), ("post_norm", (H,)), ("gate", (I, H)), ("up", (I, H)), ("down", (H, I))]
_LINEAR = [("qkv", (CD, H)), ("a", (LNH, H)), ("b", (LNH, H)), ("z", (LNH * VD, H)), ("conv", (CD, CK)),
           ("out", (H, LNH * VD)), ("A_log", (LNH,)), ("dt_bias", (LNH,)), ("norm_w", (VD,))]
_FULL = [("q", (FNH * 2 * HD, H)), ("k", (FNKV * HD, H)), ("v", (FNKV * HD, H)), ("q_norm", (HD,)),
         ("k_norm", (HD,)), ("o", (H, FNH * HD))]
_DIR_NAMES = {"in_norm": "input_layernorm", "post_norm": "post_layernorm", "gate": "mlp_gate", "up": "mlp_up",
              "down": "mlp_down", "qkv": "linear_qkv", "a": "linear_a", "b": "linear_b", "z": "linear_z",
              "conv": "linear_conv1d", "A_log": "linear_A_log", "dt_bias": "linear_dt_bias", "norm_w": "linear_norm",
              "out": "linear_out", "q": "full_q", "k": "full_k", "v": "full_v", "q_norm": "full_q_norm",
              "k_norm": "full_k_norm", "o": "full_o"}


def _read_f32(path, count=None):
    import numpy as np
    a = np.fromfile(path, dtype="<f4")
    if count is not None and a.size != count:
        raise ValueError(f"{path}: {a.size} floats, expected {count}")
    return a


def _split(flat, fields, transposed=False, offset=0):
    import numpy as np
    out = {}
    for name, shape in fields:
        n = int(np.prod(shape))
        if offset + n > flat.size:
            raise ValueError(f"flat layer too short at {name}: {flat.size} < {offset + n}")
        a = flat[offset:offset + n]
        if len(shape) == 2 and name != "conv":
            a = a.reshape(shape[::-1]).T if transposed else a.reshape(shape)
        else:
            a = a.reshape(shape)
        out[name] = np.ascontiguousarray(a, dtype=np.float32)
        offset += n
    return out, offset


def flat_layer_size(kind):
    """Floats in one flat layer: 'engine' (B, both sections) or 'linear' /
    'full' (C, one section)."""
    import numpy as np
    n = lambda fs: sum(int(np.prod(s)) for _, s in fs)
    return n(_COMMON) + {"engine": n(_LINEAR) + n(_FULL), "linear": n(_LINEAR), "full": n(_FULL)}[kind]


def layer_from_engine_flat(flat, layer_idx):
    """(B): the CudaEngine::set_layer_weights vector of one layer."""
    L, off = _split(flat, _COMMON)
    lin, off = _split(flat, _LINEAR, offset=off)
    full, off = _split(flat, _FULL, offset=off)
    if off != flat.size:
        raise ValueError(f"flat layer has {flat.size} floats, expected {off}")
    L.update(lin if is_linear_layer(layer_idx) else full)
    return L


def layer_from_export_flat(flat, layer_idx):
    """(C): one layer_XX.bin of export_real_weights.py (matrices stored [in][out])."""
    L, off = _split(flat, _COMMON, transposed=True)
    sec, off = _split(flat, _LINEAR if is_linear_layer(layer_idx) else _FULL, transposed=True, offset=off)
    if off != flat.size:
        raise ValueError(f"layer_{layer_idx:02d}.bin has {flat.size} floats, expected {off}")
    L.update(sec)
    return L


def load_dir_tree(root, num_layers=24, vocab=V_DEFAULT):
    """(A): returns (layers, final_norm, embed) as numpy float32 arrays."""
    import os
    import numpy as np
    layers = []
    for i in range(num_layers):
        pre = os.path.join(root, "language_backbone", f"layer_{i}")
        fields = _COMMON + (_LINEAR if is_linear_layer(i) else _FULL)
        layers.append({n: _read_f32(os.path.join(pre, _DIR_NAMES[n] + ".bin"), int(np.prod(s))).reshape(s)
                       for n, s in fields})
    final_norm = _read_f32(os.path.join(root, "language_backbone", "final_norm.bin"), H)
    embed = np.fromfile(os.path.join(root, "language", "embed_tokens.bin"), dtype="<f4").reshape(-1, H)
    return layers, final_norm, embed


def load_export_files(root, num_layers=24):
    """(C): weights/layer_XX.bin, norm.bin, embedding.bin; (layers, final_norm, embed)."""
    import os
    layers = [layer_from_export_flat(_read_f32(os.path.join(root, f"layer_{i:02d}.bin")), i) for i in range(num_layers)]
    final_norm = _read_f32(os.path.join(root, "norm.bin"), H)
    embed = _read_f32(os.path.join(root, "embedding.bin")).reshape(-1, H)
    return layers, final_norm, embed
