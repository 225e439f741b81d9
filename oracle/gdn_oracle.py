"""CPU oracle for the Gated DeltaNet chunked scan (numpy restatement; groundwork for its HIP kernels).

TEST INFRASTRUCTURE ONLY: only `tests/` may import this module, as the checker.  No product code calls it.

What it restates: `fast_chunk_gated_delta_rule` (modal/gdn_fast.py:37-113), the reference's copy of MaxText's
`jax_chunk_gated_delta_rule` with the precision and inverse options of gdn_fast.py:1-9.  Inputs per sequence b and
head h: q, k [T, Dk], v [T, Dv], the log-decay g [T] and the write strength beta [T].  The recurrence it computes in
chunks of C tokens (the WY form of the gated delta rule), with state S [Dk, Dv]:
    S_t = exp(g_t) (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T,      o_t = S_t^T (q_t / sqrt(Dk))
`gated_delta_recurrence` is that recurrence token by token; `gdn_chunked` is the chunked algorithm of
gdn_fast.py:63-111.  With `rounding="bf16"` the chunked form also rounds where the reference's compute dtype
(bf16, gdn_fast.py:51-55, 86, 88) rounds: q * scale, k, v and beta on entry, k * beta and v * beta, and the
intra-chunk u and w; everything else is float64 here (the reference: float32).

Pinned by tests/test_gdn_oracle.py: the chunked form equals the recurrence (float64, no rounding) for several
chunk sizes, ragged lengths (padding) and an initial state; the unit-lower-triangular inverse equals numpy's
solve and the reference's Neumann product (gdn_fast.py:21-34).
"""
from __future__ import annotations

import numpy as np

from .moe_oracle import round_bf16


def gated_delta_recurrence(q, k, v, g, beta, h0=None):
    """Token-by-token gated delta rule.  q, k [B, T, H, Dk], v [B, T, H, Dv], g, beta [B, T, H] (float64).

    Returns (o [B, T, H, Dv], final state [B, H, Dk, Dv])."""
    q, k, v, g, beta = (np.asarray(a, np.float64) for a in (q, k, v, g, beta))
    B, T, H, Dk = k.shape
    Dv = v.shape[-1]
    S = np.zeros((B, H, Dk, Dv)) if h0 is None else np.array(h0, np.float64)
    o = np.zeros((B, T, H, Dv))
    qs = q / np.sqrt(Dk)
    for t in range(T):
        kt, vt = k[:, t], v[:, t]                      # [B, H, Dk], [B, H, Dv]
        S = S * np.exp(g[:, t])[..., None, None]
        pred = np.einsum("bhk,bhkv->bhv", kt, S)       # S^T k
        S = S + beta[:, t][..., None, None] * np.einsum("bhk,bhv->bhkv", kt, vt - pred)
        o[:, t] = np.einsum("bhk,bhkv->bhv", qs[:, t], S)
    return o, S


def unit_lower_inverse(S):
    """(I + S)^-1 for strictly lower-triangular S [..., C, C] by forward substitution (float64)."""
    C = S.shape[-1]
    A = np.zeros_like(S)
    for i in range(C):
        A[..., i, :] = -np.einsum("...j,...jc->...c", S[..., i, :i], A[..., :i, :])
        A[..., i, i] += 1.0
    return A


def neumann_inverse(S):
    """The reference's INV="neumann" (gdn_fast.py:27-34): (I - S)(I + S^2)(I + S^4)... for nilpotent S."""
    C = S.shape[-1]
    eye = np.eye(C)
    A = eye - S
    P = S
    k = 2
    while k < C:
        P = P @ P
        A = A @ (eye + P)
        k *= 2
    return A


def gdn_chunked(q, k, v, g, beta, chunk=64, h0=None, rounding=None, return_uw=False):
    """fast_chunk_gated_delta_rule (modal/gdn_fast.py:37-113) without qk-norm or context parallelism.

    rounding=None: float64 throughout; "bf16": bf16 roundings at the reference's compute-dtype points.
    Returns (o [B, T, H, Dv], final state [B, H, Dk, Dv]), plus the chunk-local u [B, N, H, C, Dv] and
    w [B, N, H, C, Dk] (gdn_fast.py:88-90) with return_uw."""
    def rd(a):  # a value the reference holds in its compute dtype
        if rounding == "bf16":
            return round_bf16(np.asarray(a, np.float32)).astype(np.float64)
        return np.asarray(a, np.float64)

    B, T, H, Dk = np.shape(k)
    Dv = np.shape(v)[-1]
    scale = 1.0 / np.sqrt(Dk)
    if rounding == "bf16":
        scale = float(round_bf16(np.float32(scale)).reshape(-1)[0])
    g = np.asarray(g, np.float64)
    q = rd(rd(q) * scale)                                                           # gdn_fast.py:52, 56-57
    k, v, beta = rd(k), rd(v), rd(beta)
    pad = (chunk - T % chunk) % chunk                                               # gdn_fast.py:61-65
    if pad:
        padf = lambda a: np.concatenate([a, np.zeros((B, pad) + a.shape[2:])], axis=1)  # noqa: E731
        q, k, v, g, beta = map(padf, (q, k, v, g, beta))
    N = q.shape[1] // chunk

    def to_chunk(a):  # [B, N, H, C, D]
        return a.reshape(B, N, chunk, H, -1).transpose(0, 1, 3, 2, 4)

    qc, kc, vc = to_chunk(q), to_chunk(k), to_chunk(v)
    gc = g.reshape(B, N, chunk, H).transpose(0, 1, 3, 2)
    bc = beta.reshape(B, N, chunk, H).transpose(0, 1, 3, 2)
    gcum = np.cumsum(gc, axis=-1)                                                   # gdn_fast.py:77
    kb = rd(kc * bc[..., None])                                                     # 78 (compute dtype)
    S = kb @ kc.swapaxes(-1, -2)                                                    # 79
    lower = np.tril(np.ones((chunk, chunk), bool), k=-1)
    gd = np.where(lower, gcum[..., :, None] - gcum[..., None, :], -np.inf)
    S = np.where(lower, S * np.exp(gd), 0.0)                                        # 80-83
    A = unit_lower_inverse(S)                                                       # 85
    vb = rd(vc * bc[..., None])                                                     # 87
    u = rd(A @ vb)                                                                  # 88
    w = rd(A @ (kb * np.exp(gcum)[..., None]))                                      # 89-90
    h = np.zeros((B, H, Dk, Dv)) if h0 is None else np.array(h0, np.float64)
    incl = np.tril(np.ones((chunk, chunk), bool))
    o = np.zeros((B, N, H, chunk, Dv))
    for n in range(N):                                                              # scan_body, 99-109
        qn, kn, gg = qc[:, n], kc[:, n], gcum[:, n]
        attn_inter = (qn * np.exp(gg)[..., None]) @ h
        v_new = u[:, n] - w[:, n] @ h
        gdi = np.where(incl, gg[..., :, None] - gg[..., None, :], -np.inf)
        attn = np.where(incl, (qn @ kn.swapaxes(-1, -2)) * np.exp(gdi), 0.0)
        o[:, n] = attn_inter + attn @ v_new
        ki = kn * np.exp(gg[..., -1, None] - gg)[..., None]
        h = h * np.exp(gg[..., -1])[..., None, None] + ki.swapaxes(-1, -2) @ v_new
    o = o.transpose(0, 1, 3, 2, 4).reshape(B, N * chunk, H, Dv)[:, :T]
    return (o, h, u, w) if return_uw else (o, h)
