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

`l2norm_rows` / `l2norm_rows_bwd` restate the qk-norm branch (gdn_fast.py:43-46: MaxText's l2norm, a third-party
function absent here, y = x * rsqrt(sum(x^2) + eps) over the last axis, eps = 1e-6 as the call passes it), pinned
by the closed-form norm of its rows, scale invariance, the zero row and central finite differences of the forward.
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


def gdn_chunked_bwd(q, k, v, g, beta, do, chunk=64, h0=None, dh_final=None, rounding=None):
    """Gradients of `gdn_chunked` for the upstream gradients do [B, T, H, Dv] of o and dh_final [B, H, Dk, Dv] of the
    final state (None: 0): reverse-mode through the chunked algorithm of gdn_fast.py:63-111, which is what XLA's
    autodiff of the reference computes when the layer trains through it (installed for training at
    lightning/train_stage1.py:67-69).  The bf16 rounding points of `rounding="bf16"` round the forward values only;
    their derivative is taken as 1, as autodiff takes it for a dtype cast.

    Returns (dq, dk, dv, dg, dbeta, dh0) shaped like (q, k, v, g, beta, the initial state)."""
    def rd(a):
        if rounding == "bf16":
            return round_bf16(np.asarray(a, np.float32)).astype(np.float64)
        return np.asarray(a, np.float64)

    B, T, H, Dk = np.shape(k)
    Dv = np.shape(v)[-1]
    scale = 1.0 / np.sqrt(Dk)
    if rounding == "bf16":
        scale = float(round_bf16(np.float32(scale)).reshape(-1)[0])
    g = np.asarray(g, np.float64)
    q = rd(rd(q) * scale)
    k, v, beta = rd(k), rd(v), rd(beta)
    do = np.asarray(do, np.float64)
    C = chunk
    pad = (C - T % C) % C
    if pad:
        padf = lambda a: np.concatenate([a, np.zeros((B, pad) + a.shape[2:])], axis=1)  # noqa: E731
        q, k, v, g, beta, do = map(padf, (q, k, v, g, beta, do))
    N = q.shape[1] // C

    def to_chunk(a):
        return a.reshape(B, N, C, H, -1).transpose(0, 1, 3, 2, 4)

    qc, kc, vc, doc = to_chunk(q), to_chunk(k), to_chunk(v), to_chunk(do)
    gc = g.reshape(B, N, C, H).transpose(0, 1, 3, 2)
    bc = beta.reshape(B, N, C, H).transpose(0, 1, 3, 2)
    gg = np.cumsum(gc, axis=-1)
    strict = np.tril(np.ones((C, C), bool), k=-1)
    incl = np.tril(np.ones((C, C), bool))
    kb = rd(kc * bc[..., None])
    Gs = np.where(strict, np.exp(np.where(strict, gg[..., :, None] - gg[..., None, :], 0.0)), 0.0)
    S = (kb @ kc.swapaxes(-1, -2)) * Gs
    A = unit_lower_inverse(S)
    vb = rd(vc * bc[..., None])
    u = rd(A @ vb)
    kbg = kb * np.exp(gg)[..., None]
    w = rd(A @ kbg)
    Gi = np.where(incl, np.exp(np.where(incl, gg[..., :, None] - gg[..., None, :], 0.0)), 0.0)
    P = (qc @ kc.swapaxes(-1, -2)) * Gi
    # forward scan, keeping the state entering each chunk
    hs = np.zeros((B, N, H, Dk, Dv))
    h = np.zeros((B, H, Dk, Dv)) if h0 is None else np.array(h0, np.float64)
    for n in range(N):
        hs[:, n] = h
        gl = gg[:, n][..., -1]
        vn = u[:, n] - w[:, n] @ h
        kd = kc[:, n] * np.exp(gl[..., None] - gg[:, n])[..., None]
        h = h * np.exp(gl)[..., None, None] + kd.swapaxes(-1, -2) @ vn
    # reverse scan
    dq, dk, dv = np.zeros_like(qc), np.zeros_like(kc), np.zeros_like(vc)
    dgg, dbc = np.zeros_like(gg), np.zeros_like(bc)
    dh = np.zeros((B, H, Dk, Dv)) if dh_final is None else np.array(dh_final, np.float64)
    for n in reversed(range(N)):
        h, ggn, qn, kn = hs[:, n], gg[:, n], qc[:, n], kc[:, n]
        gl = ggn[..., -1]
        eg = np.exp(ggn)
        vn = u[:, n] - w[:, n] @ h
        kd = kn * np.exp(gl[..., None] - ggn)[..., None]
        qg = qn * eg[..., None]
        don = doc[:, n]
        # o = qg h + P v_new
        d_qg = don @ h.swapaxes(-1, -2)
        dh_prev = qg.swapaxes(-1, -2) @ don
        dP = (don @ vn.swapaxes(-1, -2)) * incl
        dvn = P[:, n].swapaxes(-1, -2) @ don
        # h_next = e^gl h + kd^T v_new
        dvn = dvn + kd @ dh
        d_kd = vn @ dh.swapaxes(-1, -2)
        dgl = np.exp(gl) * (dh * h).sum(axis=(-1, -2))
        dh_prev = dh_prev + np.exp(gl)[..., None, None] * dh
        # v_new = u - w h
        du, dw = dvn, -dvn @ h.swapaxes(-1, -2)
        dh_prev = dh_prev - w[:, n].swapaxes(-1, -2) @ dvn
        dggn = np.zeros_like(ggn)
        # P = (q k^T) * Gi
        dPr = dP * Gi[:, n]
        dq[:, n] += dPr @ kn
        dk[:, n] += dPr.swapaxes(-1, -2) @ qn
        t = dP * P[:, n]
        dggn += t.sum(axis=-1) - t.sum(axis=-2)
        # qg = q e^gg
        dq[:, n] += d_qg * eg[..., None]
        dggn += (d_qg * qg).sum(axis=-1)
        # kd = k e^(gl - gg)
        dk[:, n] += d_kd * np.exp(gl[..., None] - ggn)[..., None]
        s = (d_kd * kd).sum(axis=-1)
        dgl = dgl + s.sum(axis=-1)
        dggn -= s
        dggn[..., -1] += dgl
        # chunk-local: u = A vb, w = A kbg
        An = A[:, n]
        dA = du @ vb[:, n].swapaxes(-1, -2) + dw @ kbg[:, n].swapaxes(-1, -2)
        dvb = An.swapaxes(-1, -2) @ du
        dkbg = An.swapaxes(-1, -2) @ dw
        dkb = dkbg * eg[..., None]
        dggn += (dkbg * kbg[:, n]).sum(axis=-1)
        dS = -(An.swapaxes(-1, -2) @ dA @ An.swapaxes(-1, -2)) * strict
        dS0 = dS * Gs[:, n]
        t2 = dS * S[:, n]
        dggn += t2.sum(axis=-1) - t2.sum(axis=-2)
        dkb = dkb + dS0 @ kn
        dk[:, n] += dS0.swapaxes(-1, -2) @ kb[:, n]
        dv[:, n] += dvb * bc[:, n][..., None]
        dbc[:, n] += (dvb * vc[:, n]).sum(axis=-1) + (dkb * kn).sum(axis=-1)
        dk[:, n] += dkb * bc[:, n][..., None]
        dgg[:, n] = dggn
        dh = dh_prev
    dgc = np.flip(np.cumsum(np.flip(dgg, axis=-1), axis=-1), axis=-1)  # gg = cumsum(g) within the chunk

    def from_chunk(a):
        return a.transpose(0, 1, 3, 2, 4).reshape(B, N * C, H, -1)[:, :T]

    def from_chunk_s(a):
        return a.transpose(0, 1, 3, 2).reshape(B, N * C, H)[:, :T]

    return (from_chunk(dq) * scale, from_chunk(dk), from_chunk(dv), from_chunk_s(dgc), from_chunk_s(dbc), dh)


def l2norm_rows(x, eps=1e-6):
    """y = x * rsqrt(sum(x^2) + eps) over the last axis (gdn_fast.py:43-46, MaxText l2norm), float64; returns (y, r)
    with r = rsqrt(sum(x^2) + eps) per row."""
    x = np.asarray(x, np.float64)
    r = 1.0 / np.sqrt((x * x).sum(-1, keepdims=True) + eps)
    return x * r, r[..., 0]


def l2norm_rows_bwd(x, dy, eps=1e-6):
    """Gradient of l2norm_rows: dx = r dy - r^3 x (x . dy) per row (d/dx of x_i r with dr/dx_j = -x_j r^3)."""
    x = np.asarray(x, np.float64)
    dy = np.asarray(dy, np.float64)
    r = 1.0 / np.sqrt((x * x).sum(-1, keepdims=True) + eps)
    return r * dy - r ** 3 * x * (x * dy).sum(-1, keepdims=True)

