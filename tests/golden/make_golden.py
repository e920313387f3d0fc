"""Writes the golden vectors in this directory (run in the build container,
where oracle/_ref/libqwref.so is built from the reference's CPU sources).

Vectors:
  ref_ops.npz   inputs and outputs of the reference's own CPU operators,
                compiled from their sources by oracle/Makefile:
                  - LMHead::forward as a generic FP32 W.x
                    (src/backend/cpu/core/heads/lm_head.cpp:24-39)
                  - MLP::forward_batch
                    (src/backend/cpu/core/mlp/language_mlp.cpp:93-127)
                  - Sampler::sample greedy (src/backend/cpu/core/heads/sampler.cpp:41-43)
                    on logits with planted exact ties
                  - LinearAttention::forward, 3 tokens of one sequence from
                    non-zero conv / recurrent states
                    (src/backend/cpu/core/attention/language_linear_attn.cpp:125-257)
                  - FullAttention::forward, 6 tokens from an empty KV cache
                    (src/backend/cpu/core/attention/language_full_attn.cpp:117-216)
  quant.npz     the INT8 per-row quantize recipe
                (src/backend/cuda/kernels/mlp_cuda.cu:22-39) worked by hand
                on rows that hit each of its cases; no code computes these
                expected values.

The inputs are small (tens of KB) so the fixtures can be committed.  Run:
    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle  # noqa: E402


def ref_ops():
    R = oracle.ref_lib()
    if R is None:
        raise SystemExit("oracle/_ref/libqwref.so is not built (needs the reference tree)")
    out = {}
    # generic linear: odd M, N not a multiple of 16, K a multiple of 64
    M, N, K = 3, 50, 128
    W = oracle.normal((N, K), 11, 0.0, 0.02)
    x = oracle.normal((M, K), 12)
    y = np.empty((M, N), np.float32)
    assert R.ref_linear(W, x, y, M, N, K) == 0
    out.update(lin_W=W, lin_x=x, lin_y=y)
    # MLP block without norm/residual (MLP::forward_batch)
    M, H, I = 2, 64, 96
    Wg = oracle.normal((I, H), 21, 0.0, 0.1)
    Wu = oracle.normal((I, H), 22, 0.0, 0.1)
    Wd = oracle.normal((H, I), 23, 0.0, 0.1)
    x = oracle.normal((M, H), 24)
    y = np.empty((M, H), np.float32)
    assert R.ref_mlp(Wg, Wu, Wd, x, y, M, H, I) == 0
    out.update(mlp_Wg=Wg, mlp_Wu=Wu, mlp_Wd=Wd, mlp_x=x, mlp_y=y)
    # greedy sampler: random logits with the maximum planted at three places
    L = oracle.normal((5, 1000), 31)
    ids = []
    for r, spots in enumerate([(7,), (500, 20), (999, 998, 3), (0, 999), (123,)]):
        for s in spots:
            L[r, s] = 9.5
        ids.append(R.ref_greedy(np.ascontiguousarray(L[r]), L.shape[1]))
    out.update(greedy_logits=L, greedy_ids=np.array(ids, np.int32))
    # Gated-DeltaNet layer (small dims): projections, conv, gates, delta rule,
    # norm-gate and out projection of the reference, over 3 tokens
    H, nh, kd, vd, K, T = 64, 2, 8, 8, 4, 3
    cd = 2 * nh * kd + nh * vd
    g = dict(Wqkv=oracle.normal((cd, H), 41, 0.0, 0.2), Wa=oracle.normal((nh, H), 42, 0.0, 0.2),
             Wb=oracle.normal((nh, H), 43, 0.0, 0.2), Wz=oracle.normal((nh * vd, H), 44, 0.0, 0.2),
             conv_w=oracle.normal((cd, K), 45, 0.0, 0.5), A_log=oracle.normal((nh,), 46, 0.0, 0.5),
             dt_bias=oracle.normal((nh,), 47, 0.0, 0.5), norm_w=1.0 + oracle.normal((vd,), 48, 0.0, 0.1),
             Wout=oracle.normal((H, nh * vd), 49, 0.0, 0.2), conv_state=oracle.normal((cd, K - 1), 50),
             rec_state=oracle.normal((nh, kd * vd), 51, 0.0, 0.3), x=oracle.normal((T, H), 52))
    y, cs, rs = oracle.ref_linear_attn(g["x"], g["Wqkv"], g["Wa"], g["Wb"], g["Wz"], g["conv_w"], g["A_log"],
                                       g["dt_bias"], g["norm_w"], g["Wout"], g["conv_state"], g["rec_state"],
                                       nh, kd, vd)
    out.update({"gdn_" + k: v for k, v in g.items()})
    out.update(gdn_y=y, gdn_conv_state_out=cs, gdn_rec_state_out=rs)
    # gated full attention (small dims, GQA 4:2, head dim 16, rotary 4 dims,
    # theta 100 so the rotations are large): 6 tokens from an empty cache
    H, nh, nkv, hd, T = 64, 4, 2, 16, 6
    f = dict(Wq=oracle.normal((nh * hd * 2, H), 61, 0.0, 0.2), Wk=oracle.normal((nkv * hd, H), 62, 0.0, 0.2),
             Wv=oracle.normal((nkv * hd, H), 63, 0.0, 0.2), qn=oracle.normal((hd,), 64, 0.0, 0.1),
             kn=oracle.normal((hd,), 65, 0.0, 0.1), Wo=oracle.normal((H, nh * hd), 66, 0.0, 0.2),
             x=oracle.normal((T, H), 67))
    y = oracle.ref_full_attn(f["x"], f["Wq"], f["Wk"], f["Wv"], f["qn"], f["kn"], f["Wo"], nh, nkv, hd, hd,
                             theta=100.0, partial=0.25)
    out.update({"fa_" + k: v for k, v in f.items()})
    out.update(fa_y=y)
    np.savez_compressed(os.path.join(HERE, "ref_ops.npz"), **out)


def quant():
    # Each row's max |w| fixes s = max/127 (s <= 1e-8 -> 1), then
    # q = clamp(roundf(w / s), -127, 127) with halves rounded away from zero.
    W = np.array([
        [127.0, -63.5, 0.5, -0.5, 1.5, -2.5, 0.0, 126.5],   # s = 1: ties round away
        [254.0, 1.0, -3.0, 5.0, -254.0, 0.0, 2.0, -1.0],    # s = 2: 0.5 -> 1, -1.5 -> -2, 2.5 -> 3
        [1e-9, -5e-10, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0],       # max < 1e-8*127 -> s = 1, q = 0
        [0.0] * 8,                                          # all zero -> s = 1
        [-12.7, 6.35, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0],        # s = 0.1 (as FP32 division)
    ], np.float32)
    s = np.array([1.0, 2.0, 1.0, 1.0, np.float32(12.7) / np.float32(127.0)], np.float32)
    q = np.array([
        [127, -64, 1, -1, 2, -3, 0, 127],
        [127, 1, -2, 3, -127, 0, 1, -1],
        [0, 0, 0, 0, 0, 0, 0, 0],
        [0, 0, 0, 0, 0, 0, 0, 0],
        [-127, 64, 0, 0, 0, 0, 0, 0],
    ], np.int8)
    np.savez_compressed(os.path.join(HERE, "quant.npz"), W=W, s=s, q=q)


if __name__ == "__main__":
    ref_ops()
    quant()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
