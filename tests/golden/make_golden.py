"""Writes the golden fixtures in tests/golden/*.npz.

The reference ships no vectors for this path (its only test,
core/myFlashAttn.py:26-64, compares two live implementations), so the expected
outputs here come from a float64 numpy implementation written row by row,
independently of oracle/ (different route through the maths: the backward
uses D_i = sum_j P_ij dP_ij instead of rowsum(dO * O), and the loops run per
row / per key).  Inputs are seeded and stored in the fixture.

Run:  python tests/golden/make_golden.py
"""
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def rope_tables(D, S, base=10000.0):
    # fp32 angles as core/position_embeddings.py:19,34-40 builds them
    freqs = (1.0 / (np.float32(base) ** (np.arange(0, D, 2, dtype=np.float32) / np.float32(D))))
    freqs = freqs.astype(np.float32)
    t = np.arange(S, dtype=np.float32)
    th = np.outer(t, freqs).astype(np.float32)
    return np.cos(th).astype(np.float32), np.sin(th).astype(np.float32)


def rope_rows(x, c, s, inverse=False):
    """x [S,B,H,D] float64; pair-by-pair loop over i."""
    out = np.empty_like(x)
    D = x.shape[-1]
    for i in range(D // 2):
        e, o = x[..., 2 * i], x[..., 2 * i + 1]
        ci = c[: x.shape[0], i][:, None, None]
        si = s[: x.shape[0], i][:, None, None]
        if inverse:
            out[..., 2 * i] = e * ci + o * si
            out[..., 2 * i + 1] = o * ci - e * si
        else:
            out[..., 2 * i] = e * ci - o * si
            out[..., 2 * i + 1] = e * si + o * ci
    return out


def attn_head(q, k, v, do, causal):
    """One head, float64, row loops.  Returns o, lse, dq, dk, dv."""
    S, D = q.shape
    scale = 1.0 / math.sqrt(D)
    o = np.zeros((S, D))
    lse = np.zeros(S)
    P = np.zeros((S, S))
    for i in range(S):
        n = i + 1 if causal else S
        sc = np.array([scale * float(np.dot(q[i], k[j])) for j in range(n)])
        mx = sc.max()
        w = np.exp(sc - mx)
        tot = w.sum()
        P[i, :n] = w / tot
        lse[i] = mx + math.log(tot)
        o[i] = (P[i, :n, None] * v[:n]).sum(0)
    dv = np.zeros((S, D))
    for j in range(S):
        dv[j] = (P[:, j, None] * do).sum(0)
    dP = np.array([[float(np.dot(do[i], v[j])) for j in range(S)] for i in range(S)])
    Drow = (P * dP).sum(1)
    dS = P * (dP - Drow[:, None])
    dq = np.zeros((S, D))
    dk = np.zeros((S, D))
    for i in range(S):
        dq[i] = scale * (dS[i, :, None] * k).sum(0)
    for j in range(S):
        dk[j] = scale * (dS[:, j, None] * q).sum(0)
    return o, lse, dq, dk, dv


def attn_case(name, B, H, S, D, causal, seed, std=1.0, with_rope=True):
    rng = np.random.default_rng(seed)
    # model layout [S,B,H,D] for the RoPE stage, attention layout [B,H,S,D]
    q_sbhd = (rng.standard_normal((S, B, H, D)) * std).astype(np.float32)
    k_sbhd = (rng.standard_normal((S, B, H, D)) * std).astype(np.float32)
    v = (rng.standard_normal((B, H, S, D)) * std).astype(np.float32)
    do = rng.standard_normal((B, H, S, D)).astype(np.float32)
    c, s = rope_tables(D, S)
    if with_rope:
        qr = rope_rows(q_sbhd.astype(np.float64), c.astype(np.float64), s.astype(np.float64))
        kr = rope_rows(k_sbhd.astype(np.float64), c.astype(np.float64), s.astype(np.float64))
    else:
        qr, kr = q_sbhd.astype(np.float64), k_sbhd.astype(np.float64)
    q = qr.transpose(1, 2, 0, 3)
    k = kr.transpose(1, 2, 0, 3)
    res = {n: np.zeros((B, H, S, D)) for n in ("o", "dq", "dk", "dv")}
    res["lse"] = np.zeros((B, H, S))
    for b in range(B):
        for h in range(H):
            o, lse, dq, dk, dv = attn_head(q[b, h], k[b, h], v[b, h].astype(np.float64),
                                           do[b, h].astype(np.float64), causal)
            res["o"][b, h], res["lse"][b, h] = o, lse
            res["dq"][b, h], res["dk"][b, h], res["dv"][b, h] = dq, dk, dv
    np.savez_compressed(
        os.path.join(HERE, f"{name}.npz"),
        q_sbhd=q_sbhd, k_sbhd=k_sbhd, v=v, do=do, cos=c, sin=s,
        causal=np.array(causal), with_rope=np.array(with_rope),
        q_rot=q.astype(np.float32), k_rot=k.astype(np.float32),
        **{n: a.astype(np.float32) for n, a in res.items()})


def rope_case(name, S, B, H, D, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((S, B, H, D)).astype(np.float32)
    c, s = rope_tables(D, S)
    fwd = rope_rows(x.astype(np.float64), c.astype(np.float64), s.astype(np.float64))
    inv = rope_rows(x.astype(np.float64), c.astype(np.float64), s.astype(np.float64), True)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), x=x, cos=c, sin=s,
                        fwd=fwd.astype(np.float32), inv=inv.astype(np.float32))


if __name__ == "__main__":
    # config-1 shape family (fp32, causal, RoPE on q/k), reduced to 1 head x 128
    attn_case("attn_causal_s128_d64", B=1, H=1, S=128, D=64, causal=True, seed=1)
    attn_case("attn_noncausal_s64_d32", B=2, H=1, S=64, D=32, causal=False, seed=2)
    attn_case("attn_causal_ragged_s45_d16", B=1, H=1, S=45, D=16, causal=True, seed=3)
    attn_case("attn_causal_s64_d128", B=1, H=1, S=64, D=128, causal=True, seed=4, std=0.5)
    rope_case("rope_s24_b2_h3_d16", S=24, B=2, H=3, D=16, seed=5)
    print("fixtures written to", HERE)
