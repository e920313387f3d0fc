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
                 kv_int8=True):
        import torch
        self.qw, self.ctx, self.B = qw, ctx, batch
        fmt = qw.WFMT_BF16 if fmt is None else fmt
        lm_fmt = qw.WFMT_BF16 if lm_fmt is None else lm_fmt
        dev = "cuda"
        self.act = torch.float32 if fmt == qw.WFMT_F32 else torch.bfloat16
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

    def step(self, stream=None):
        """One greedy token for every sequence: ids <- next ids, positions += 1."""
        qw, ctx, x, row = self.qw, self.ctx, self.x, self.row
        qw.embedding_gather(ctx, self.embed, self.ids, x, stream=stream)
        for P in self.layers:
            if P["linear"]:
                r = row[:, :LIN_IN]
                qw.linear(ctx, P["in"], x, r, gamma=P["in_norm"], stream=stream)
                qw.gdn_decode(ctx, P["conv"], P["A_log"], P["dt_bias"], P["norm_w"], r[:, :CD],
                              r[:, CD:CD + LNH * VD], r[:, CD + LNH * VD:CD + LNH * VD + LNH],
                              r[:, CD + LNH * VD + LNH:], P["cs"], P["rs"], self.core, LNH, ld_in=row.stride(0),
                              stream=stream)
            else:
                r = row[:, :FULL_IN]
                qw.linear(ctx, P["in"], x, r, gamma=P["in_norm"], stream=stream)
                qw.attn_forward(ctx, P["q_norm"], P["k_norm"], P["cache"], self.pos, r[:, 0:], r[:, HD:],
                                r[:, FNH * 2 * HD:], r[:, FNH * 2 * HD + FNKV * HD:], self.core, tokens=1,
                                q_head_stride=2 * HD, ld_in=row.stride(0), max_len=self.capacity, stream=stream)
            qw.linear(ctx, P["out"], self.core, x, residual=x, stream=stream)
            qw.mlp_fused(ctx, P["gateup"], P["down"], x, x, gamma=P["post_norm"], residual=x, stream=stream)
        qw.rmsnorm(ctx, x, self.final_norm, self.xn, stream=stream)
        qw.lmhead_argmax(ctx, self.E, self.xn, self.ids, stream=stream)
        qw.positions_add(ctx, self.pos, 1, stream=stream)
