"""TEST INFRASTRUCTURE — independent float64 restatements used to pin the C++ oracle.

Written from the mathematics of the recurrences, sharing no code with
`cpu_ref.cpp`. Each uses a different evaluation structure from the C++ file,
so a transcription slip there (a dropped term, a wrong index, a transposed
operand, the wrong trapezoid neighbour under reverse) shows up as a mismatch:

* `m1_scan`: vectorised over (batch, channel), with reverse implemented as
  flip -> forward -> flip (the reference's definition, lib.rs:107-126).
* `m3_siso_scan`: the sequential form with reverse as flip -> forward -> flip
  applied AFTER the rotation (tests/reference/mamba3_ref.py:216-267 states why
  the order matters).
* `m3_siso_dense`: the O(L^2) dual (attention-like) form of the same SISO
  recurrence — no state matrix at all.
* `m3_mimo_scan`: the rank-r sequential form, einsum-free.
* `m3_mixer`: the Mamba-3 mixer (apps/mamba3_lm/block.py:146-199) around the
  sequential scans: in_proj, the split, `heavy_tail`, softplus, `rms_norm`, Q <- C /
  K <- B, the head-shared angles, out_proj.
* `m3_noncausal_dense`: the non-causal (and, with causal=True, the causal) O(L^2)
  mask form with every weight a running product of decays (no cumsum), and
  `m3_same_step`, the same-step term from UNROTATED q/k, so that
  forward + backward - same-step == dense also pins RoPE's invariance of q_t . k_t.

Only for small shapes: these are loops in numpy.
"""

import numpy as np


def softplus(x):
    x = np.asarray(x, np.float64)
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def silu(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def sigmoid(x):
    x = np.asarray(x, np.float64)
    return 0.5 * (1.0 + np.tanh(0.5 * x))


def m1_scan(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
            reverse=False, h0=None):
    """Mamba-1 selective scan in float64 -> (out (b,d,l), last_state (b,d,n))."""
    u = np.asarray(u, np.float64)
    delta = np.asarray(delta, np.float64)
    A = np.asarray(A, np.float64)
    B = np.asarray(B, np.float64)
    C = np.asarray(C, np.float64)
    b, d, L = u.shape
    n = A.shape[1]
    if B.ndim == 3:
        B, C = B[:, None], C[:, None]
    g = B.shape[1]
    # channel d reads group d // (d_total / g) (lib.rs:82-83)
    gidx = np.arange(d) // (d // g)
    Bd = B[:, gidx]  # (b, d, n, L)
    Cd = C[:, gidx]
    if delta_bias is not None:
        delta = delta + np.asarray(delta_bias, np.float64)[None, :, None]
    if delta_softplus:
        delta = softplus(delta)
    if reverse:
        u, delta = u[..., ::-1], delta[..., ::-1]
        Bd, Cd = Bd[..., ::-1], Cd[..., ::-1]
        zz = None if z is None else np.asarray(z, np.float64)[..., ::-1]
    else:
        zz = None if z is None else np.asarray(z, np.float64)
    h = np.zeros((b, d, n)) if h0 is None else np.array(h0, np.float64)
    out = np.empty((b, d, L))
    for t in range(L):
        h = np.exp(delta[:, :, t, None] * A[None]) * h \
            + (delta[:, :, t] * u[:, :, t])[..., None] * Bd[:, :, :, t]
        out[:, :, t] = (h * Cd[:, :, :, t]).sum(-1)
    if D is not None:
        out = out + u * np.asarray(D, np.float64)[None, :, None]
    if zz is not None:
        out = out * silu(zz)
    if reverse:
        out = out[..., ::-1]
    return np.ascontiguousarray(out), h


def _rope_interleaved(x, cos, sin):
    a, b = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = a * cos - b * sin
    out[..., 1::2] = a * sin + b * cos
    return out


def _rope_split(x, cos, sin):
    half = x.shape[-1] // 2
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * cos - b * sin, a * sin + b * cos], axis=-1)


def _m3_prep(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, z, heads, rope):
    """Bias, rotate and expand q/k to per-head (b, l, [r,] h, dqk) in float64."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    g = q.shape[-2]
    hidx = np.arange(heads) // (heads // g)
    q = q[..., hidx, :] + np.asarray(q_bias, np.float64)
    k = k[..., hidx, :] + np.asarray(k_bias, np.float64)
    cos = np.asarray(cos, np.float64)
    sin = np.asarray(sin, np.float64)
    if q.ndim == 5:  # (b, l, r, h, dqk): angles shared across rank
        cos, sin = cos[:, :, None], sin[:, :, None]
    return rope(q, cos, sin), rope(k, cos, sin)


def _gates(adt, dt, trap):
    dt = np.asarray(dt, np.float64)
    lam = sigmoid(trap)
    gamma = dt * lam
    shifted = np.zeros_like(gamma)
    shifted[..., :-1] = dt[..., 1:] * (1.0 - lam[..., 1:])
    return gamma, gamma + shifted, np.exp(np.asarray(adt, np.float64))


def m3_siso_scan(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, D=None, z=None,
                 reverse=False):
    """Mamba-3 SISO in float64 -> (out time-major (b,l,h,dv), last_state (b,h,dv,dqk)).

    q, k (b, l, g, dqk) with g dividing h; interleaved RoPE on (q + bias).
    """
    v = np.asarray(v, np.float64)
    b, L, h, dv = v.shape
    q, k = _m3_prep(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, z, h,
                    _rope_interleaved)
    adt, dt, trap = (np.asarray(x, np.float64) for x in (adt, dt, trap))
    zz = None if z is None else np.asarray(z, np.float64)
    if reverse:
        q, k, v = q[:, ::-1], k[:, ::-1], v[:, ::-1]
        adt, dt, trap = adt[..., ::-1], dt[..., ::-1], trap[..., ::-1]
        zz = None if zz is None else zz[:, ::-1]
    gamma, scale, alpha = _gates(adt, dt, trap)
    dqk = q.shape[-1]
    S = np.zeros((b, h, dv, dqk))
    out = np.empty((b, L, h, dv))
    Dv = np.zeros(h) if D is None else np.asarray(D, np.float64)
    for t in range(L):
        qt, kt, vt = q[:, t], k[:, t], v[:, t]  # (b,h,dqk), (b,h,dqk), (b,h,dv)
        y = alpha[:, :, t, None] * (S * qt[:, :, None, :]).sum(-1)
        coef = Dv[None] + gamma[:, :, t] * (qt * kt).sum(-1)
        out[:, t] = y + coef[..., None] * vt
        S = alpha[:, :, t, None, None] * S \
            + scale[:, :, t, None, None] * vt[..., None] * kt[..., None, :]
    if zz is not None:
        out = out * silu(zz)
    if reverse:
        out = out[:, ::-1]
    return np.ascontiguousarray(out), S


def m3_siso_dense(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, D=None, z=None):
    """Forward Mamba-3 SISO via the dual form, no state matrix.

    y_t = sum_{s<=t} W_ts (q_t . k_s) v_s + D v_t, with
    W_ts = exp(sum_{s<u<=t} adt_u) * scale_s for s < t and W_tt = gamma_t.
    """
    v = np.asarray(v, np.float64)
    b, L, h, dv = v.shape
    q, k = _m3_prep(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, z, h,
                    _rope_interleaved)
    gamma, scale, _ = _gates(adt, dt, trap)
    c = np.cumsum(np.asarray(adt, np.float64), axis=-1)  # (b, h, L)
    G = np.einsum("bthn,bshn->bhts", q, k)  # (b, h, t, s)
    decay = np.exp(c[..., :, None] - c[..., None, :])
    W = np.where(np.tril(np.ones((L, L)), -1)[None, None] > 0,
                 decay * scale[..., None, :], 0.0)
    idx = np.arange(L)
    W[..., idx, idx] = gamma
    out = np.einsum("bhts,bshp->bthp", G * W, v)
    if D is not None:
        out = out + np.asarray(D, np.float64)[None, None, :, None] * v
    if z is not None:
        out = out * silu(z)
    return out


def m3_same_step(q, k, v, dt, trap, q_bias, k_bias, D=None, z=None):
    """The s == t term of Mamba-3 SISO, (D + gamma_t (q_t . k_t)) v_t, gated
    (python/arm_scan/mamba3_noncausal.py:47-86). q_t . k_t from q + bias, k + bias
    WITHOUT rotation: RoPE turns both by the same angle at one position."""
    v = np.asarray(v, np.float64)
    b, L, h, dv = v.shape
    g = q.shape[-2]
    hidx = np.arange(h) // (h // g)
    qb = np.asarray(q, np.float64)[..., hidx, :] + np.asarray(q_bias, np.float64)
    kb = np.asarray(k, np.float64)[..., hidx, :] + np.asarray(k_bias, np.float64)
    gamma = np.asarray(dt, np.float64) * sigmoid(trap)  # (b, h, L)
    coef = gamma.transpose(0, 2, 1) * (qb * kb).sum(-1)  # (b, L, h)
    if D is not None:
        coef = coef + np.asarray(D, np.float64)
    out = coef[..., None] * v
    return out if z is None else out * silu(z)


def m3_noncausal_dense(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, D=None, z=None,
                       causal=False):
    """Mamba-3 SISO over every position (python/arm_scan/mamba3_noncausal.py:101-178)
    in float64: y_t = sum_s W[t, s] (q_t . k_s) v_s + D v_t, gated, with

      W[t, s] = alpha_{s+1} ... alpha_t * scale_s          s < t (forward trapezoid,
                                                           scale_s = gamma_s + dt_{s+1}(1 - lam_{s+1}))
      W[t, t] = gamma_t
      W[t, s] = alpha_t ... alpha_{s-1} * scale'_s         s > t (backward traversal,
                                                           scale'_s = gamma_s + dt_{s-1}(1 - lam_{s-1}))

    alpha = exp(adt), lam = sigmoid(trap); the s > t half is dropped when causal.
    """
    v = np.asarray(v, np.float64)
    b, L, h, dv = v.shape
    q, k = _m3_prep(q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, z, h,
                    _rope_interleaved)
    dt = np.asarray(dt, np.float64)
    lam = sigmoid(trap)
    alpha = np.exp(np.asarray(adt, np.float64))
    gamma = dt * lam
    scale_f = gamma.copy()
    scale_f[..., :-1] += dt[..., 1:] * (1.0 - lam[..., 1:])
    scale_b = gamma.copy()
    scale_b[..., 1:] += dt[..., :-1] * (1.0 - lam[..., :-1])
    W = np.zeros((b, h, L, L))
    for t in range(L):
        W[..., t, t] = gamma[..., t]
        decay = np.ones((b, h))
        for s in range(t - 1, -1, -1):
            decay = decay * alpha[..., s + 1]
            W[..., t, s] = decay * scale_f[..., s]
        if not causal:
            decay = np.ones((b, h))
            for s in range(t + 1, L):
                decay = decay * alpha[..., s - 1]
                W[..., t, s] = decay * scale_b[..., s]
    G = np.einsum("bthn,bshn->bhts", q, k)
    out = np.einsum("bhts,bshp->bthp", G * W, v)
    if D is not None:
        out = out + np.asarray(D, np.float64)[None, None, :, None] * v
    if z is not None:
        out = out * silu(z)
    return out


def m3_mimo_scan(q, k, v, adt, dt, trap, q_bias, k_bias, psi, zeta, phi, cos, sin,
                 D=None, z=None, reverse=False):
    """Mamba-3 MIMO in float64 -> (out time-major (b,l,h,dv), last_state).

    q, k (b, l, r, g, dqk); split-halves RoPE; x_r = psi_r * v; gate per rank
    silu(z * zeta_r); phi reduces the rank axis.
    """
    v = np.asarray(v, np.float64)
    b, L, h, dv = v.shape
    q, k = _m3_prep(q, k, v, adt, dt, trap, q_bias.transpose(1, 0, 2),
                    k_bias.transpose(1, 0, 2), cos, sin, z, h, _rope_split)
    # q, k: (b, l, r, h, dqk); biases were given (h, r, dqk)
    adt, dt, trap = (np.asarray(x, np.float64) for x in (adt, dt, trap))
    psi, zeta, phi = (np.asarray(x, np.float64).transpose(1, 0, 2) for x in (psi, zeta, phi))
    x = v[:, :, None] * psi[None, None]  # (b, l, r, h, dv)
    zz = None if z is None else np.asarray(z, np.float64)
    if reverse:
        q, k, x = q[:, ::-1], k[:, ::-1], x[:, ::-1]
        adt, dt, trap = adt[..., ::-1], dt[..., ::-1], trap[..., ::-1]
        zz = None if zz is None else zz[:, ::-1]
    gamma, scale, alpha = _gates(adt, dt, trap)
    r = q.shape[2]
    dqk = q.shape[-1]
    S = np.zeros((b, h, dv, dqk))
    out = np.zeros((b, L, h, dv))
    Dv = np.zeros(h) if D is None else np.asarray(D, np.float64)
    for t in range(L):
        qt, kt, xt = q[:, t], k[:, t], x[:, t]  # (b, r, h, *)
        acc = np.empty((b, r, h, dv))
        for ro in range(r):
            y = (S * qt[:, ro, :, None, :]).sum(-1)  # (b, h, dv)
            dsum = np.zeros((b, h, dv))
            for ri in range(r):
                dsum += (qt[:, ro] * kt[:, ri]).sum(-1)[..., None] * xt[:, ri]
            acc[:, ro] = alpha[:, :, t, None] * y + gamma[:, :, t, None] * dsum \
                + Dv[None, :, None] * xt[:, ro]
        upd = np.zeros((b, h, dv, dqk))
        for ri in range(r):
            upd += xt[:, ri][..., None] * kt[:, ri][..., None, :]
        S = alpha[:, :, t, None, None] * S + scale[:, :, t, None, None] * upd
        for ro in range(r):
            term = acc[:, ro] * phi[ro][None]
            if zz is not None:
                term = term * silu(zz[:, t] * zeta[ro][None])
            out[:, t] += term
    if reverse:
        out = out[:, ::-1]
    return np.ascontiguousarray(out), S


def causal_conv1d(x, w, bias=None, silu_act=False):
    """Depthwise causal convolution (transformers modeling_mamba.py causal_conv1d_fn) in
    float64: y[b, d, t] = bias[d] + sum_k w[d, k] x[b, d, t - K + 1 + k], x[t < 0] = 0,
    through numpy's full convolution per row."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    b, d, L = x.shape
    y = np.empty((b, d, L))
    for j in range(d):
        for i in range(b):
            y[i, j] = np.convolve(x[i, j], w[j, ::-1])[:L]
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :, None]
    return silu(y) if silu_act else y


def heavy_tail(x):
    """1 + x for x >= 0, 1 / (1 - x) below (apps/mamba3_lm/block.py:52-62)."""
    x = np.asarray(x, np.float64)
    return np.where(x >= 0, 1.0 + x, 1.0 / (1.0 - np.minimum(x, 0.0)))


def rms_norm(x, w, eps):
    """x / sqrt(mean(x^2) + eps) * w over the last axis (block.py:65-82)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def m3_mixer(u, p, heads, headdim, d_state, rank, groups, n_angles, a_floor, eps=1e-5):
    """The Mamba-3 mixer forward (apps/mamba3_lm/block.py:146-199) in float64.

    u (b, l, d_model); p: in_proj (d_in_proj, d_model), out_proj (d_model, d_inner),
    dt_bias, D (h), B_bias, C_bias (h, r, n), B_norm, C_norm (n) and, for MIMO,
    mimo_x / mimo_z / mimo_o (h, r, headdim). Projection columns in the checkpoint's
    order [z, x, B, C, dd_dt, dd_A, trap, angles] (block.py:113-118).
    """
    import oracle

    u = np.asarray(u, np.float64)
    b, L, _ = u.shape
    d_inner, bc = heads * headdim, rank * groups * d_state
    proj = u @ np.asarray(p["in_proj"], np.float64).T
    sizes = [d_inner, d_inner, bc, bc, heads, heads, heads, n_angles]
    z, x, B, C, dd_dt, dd_A, trap, ang = np.split(proj, np.cumsum(sizes)[:-1], axis=-1)
    z = z.reshape(b, L, heads, headdim)
    x = x.reshape(b, L, heads, headdim)
    B = rms_norm(B.reshape(b, L, rank, groups, d_state), p["B_norm"], eps)
    C = rms_norm(C.reshape(b, L, rank, groups, d_state), p["C_norm"], eps)
    A = np.minimum(-heavy_tail(dd_A), -a_floor)
    DT = softplus(dd_dt + np.asarray(p["dt_bias"], np.float64))
    ADT = (A * DT).transpose(0, 2, 1)
    DT = DT.transpose(0, 2, 1)
    trap = trap.transpose(0, 2, 1)
    ang = np.broadcast_to(ang[:, :, None, :], (b, L, heads, n_angles))
    cos, sin = oracle.angles_to_cos_sin(ang, DT, d_state // 2)
    if "mimo_x" not in p:
        y, _ = m3_siso_scan(C[:, :, 0], B[:, :, 0], x, ADT, DT, trap, p["C_bias"][:, 0],
                            p["B_bias"][:, 0], cos, sin, D=p["D"], z=z)
    else:
        y, _ = m3_mimo_scan(C, B, x, ADT, DT, trap, p["C_bias"], p["B_bias"], p["mimo_x"],
                            p["mimo_z"], p["mimo_o"], cos, sin, D=p["D"], z=z)
    return y.reshape(b, L, d_inner) @ np.asarray(p["out_proj"], np.float64).T
