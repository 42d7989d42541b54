"""Float64 restatement of the three recurrences, written from their mathematical
definitions, with every derivative taken by torch autograd (test infrastructure).

Used to pin the CPU oracle independently of the reference's code: the values
come from the recurrences below, the marginals / parameter gradients from one
backward pass, Hessian-vector products and parameter Jacobians from a double
backward.  Cells are Python objects (``None`` = unreachable), so sizes are kept
to a few dozen cells.

Recurrences (1-based DP indices, s / c indexed from 0):
  linear SW   a[0,0] = 0, other row/column-0 cells unreachable;
              a[i,j] = LSE_T(a[i-1,j-1] + s (i>1, j>1), a[i-1,j] + gap (i>1),
                             a[i,j-1] + gap (j>1), s);
              S = LSE_T(a[0,0], a[i,j] for all i, j >= 1).
  affine SW   M[0,0] = 0;  M = LSE_T(M|I|D[i-1,j-1] + s (i>1, j>1), s);
              I = LSE_T(M[i-1,j] + open, I[i-1,j] + ext) (i>1);
              D = LSE_T(M[i,j-1] + open, D[i,j-1] + ext) (j>1);
              S = LSE_T(M[0,0], every reachable M, I, D).
  DTW         a[0,0] = 0;  a[i,j] = c + softmin_T(a[i-1,j-1], a[i-1,j], a[i,j-1])
              over reachable in-band predecessors; S = a[L1,L2] (+inf if
              unreachable).  Band: |j - i*L2/L1| <= bandwidth (none if < 0).
LSE_T(x) = T log sum exp(x / T); softmin_T(x) = -LSE_T(-x).
"""
from __future__ import annotations

import math

import torch

D = torch.float64


def _lse(terms, T):
    return T * torch.logsumexp(torch.stack(terms) / T, 0)


def sw_value(s, gap, T):
    L1, L2 = s.shape
    a = [[None] * (L2 + 1) for _ in range(L1 + 1)]
    a[0][0] = torch.zeros((), dtype=D)
    cells = [a[0][0]]
    for i in range(1, L1 + 1):
        for j in range(1, L2 + 1):
            x = s[i - 1, j - 1]
            t = [x]
            if i > 1 and j > 1:
                t.append(a[i - 1][j - 1] + x)
            if i > 1:
                t.append(a[i - 1][j] + gap)
            if j > 1:
                t.append(a[i][j - 1] + gap)
            a[i][j] = _lse(t, T)
            cells.append(a[i][j])
    return _lse(cells, T)


def nw_value(s, gap, T):
    """Global alignment: alpha[0,0] = 0, alpha[i,0] = i*gap, alpha[0,j] = j*gap,
    alpha[i,j] = LSE(diag + s, up + gap, left + gap); the value is alpha[L1, L2]."""
    L1, L2 = s.shape
    a = [[None] * (L2 + 1) for _ in range(L1 + 1)]
    a[0][0] = torch.zeros((), dtype=D) * gap
    for i in range(1, L1 + 1):
        a[i][0] = i * gap
    for j in range(1, L2 + 1):
        a[0][j] = j * gap
    for i in range(1, L1 + 1):
        for j in range(1, L2 + 1):
            a[i][j] = _lse([a[i - 1][j - 1] + s[i - 1, j - 1], a[i - 1][j] + gap,
                            a[i][j - 1] + gap], T)
    return a[L1][L2]


def swa_value(s, go, ge, T):
    L1, L2 = s.shape
    M = [[None] * (L2 + 1) for _ in range(L1 + 1)]
    I = [[None] * (L2 + 1) for _ in range(L1 + 1)]
    Dm = [[None] * (L2 + 1) for _ in range(L1 + 1)]
    M[0][0] = torch.zeros((), dtype=D)
    cells = [M[0][0]]
    for i in range(1, L1 + 1):
        for j in range(1, L2 + 1):
            x = s[i - 1, j - 1]
            t = [x]
            if i > 1 and j > 1:
                t += [v + x for v in (M[i - 1][j - 1], I[i - 1][j - 1], Dm[i - 1][j - 1])
                      if v is not None]
            M[i][j] = _lse(t, T)
            if i > 1:
                t = [v for v in (M[i - 1][j] + go,
                                 None if I[i - 1][j] is None else I[i - 1][j] + ge)
                     if v is not None]
                I[i][j] = _lse(t, T)
            if j > 1:
                t = [v for v in (M[i][j - 1] + go,
                                 None if Dm[i][j - 1] is None else Dm[i][j - 1] + ge)
                     if v is not None]
                Dm[i][j] = _lse(t, T)
            cells += [v for v in (M[i][j], I[i][j], Dm[i][j]) if v is not None]
    return _lse(cells, T)


def in_band(i, j, L1, L2, bw):
    if bw < 0 or L1 == 0 or L2 == 0:
        return True
    return abs(j - i * L2 / L1) <= bw


def dtw_value(c, T, bw=-1):
    L1, L2 = c.shape
    a = [[None] * (L2 + 1) for _ in range(L1 + 1)]
    a[0][0] = torch.zeros((), dtype=D)
    for i in range(1, L1 + 1):
        for j in range(1, L2 + 1):
            if not in_band(i, j, L1, L2, bw):
                continue
            preds = [a[p][q] for p, q in ((i - 1, j - 1), (i - 1, j), (i, j - 1))
                     if a[p][q] is not None and in_band(p, q, L1, L2, bw)]
            if preds:
                a[i][j] = c[i - 1, j - 1] - _lse([-p for p in preds], T)
    if a[L1][L2] is None:
        return torch.tensor(math.inf, dtype=D)
    return a[L1][L2]


# ------------------------------------------------------------------ derivatives

def _leaf(x):
    return torch.as_tensor(x, dtype=D).clone().requires_grad_(True)


def _grads(value_fn, x, params):
    """value, dS/dx, [dS/dparam]."""
    x = _leaf(x)
    ps = [_leaf(p) for p in params]
    S = value_fn(x, *ps)
    if not S.requires_grad:            # empty problem: constant value
        return S.detach(), torch.zeros_like(x), [torch.zeros((), dtype=D) for _ in ps]
    g = torch.autograd.grad(S, [x] + ps, allow_unused=True)
    g = [torch.zeros_like(v) if gi is None else gi for gi, v in zip(g, [x] + ps)]
    return S.detach(), g[0], g[1:]


def _hvp(value_fn, x, params, V):
    x = _leaf(x)
    ps = [torch.as_tensor(p, dtype=D) for p in params]
    S = value_fn(x, *ps)
    if not S.requires_grad:
        return torch.zeros_like(x)
    (P,) = torch.autograd.grad(S, x, create_graph=True, allow_unused=True)
    if P is None or not P.requires_grad:
        return torch.zeros_like(x)
    (H,) = torch.autograd.grad((P * torch.as_tensor(V, dtype=D)).sum(), x, allow_unused=True)
    return torch.zeros_like(x) if H is None else H


def _param_jac(value_fn, x, params, k):
    """d(dS/dx)/dparam_k = d/dx (dS/dparam_k)."""
    x = _leaf(x)
    ps = [_leaf(p) for p in params]
    S = value_fn(x, *ps)
    if not S.requires_grad:
        return torch.zeros_like(x)
    (gk,) = torch.autograd.grad(S, ps[k], create_graph=True, allow_unused=True)
    if gk is None or not gk.requires_grad:
        return torch.zeros_like(x)
    (J,) = torch.autograd.grad(gk, x, allow_unused=True)
    return torch.zeros_like(x) if J is None else J


def _batched(fn, x, lengths, *extra):
    """Apply a per-element function to the valid [:l1, :l2] block of each element,
    zero elsewhere."""
    import numpy as np
    x = np.asarray(x, dtype=np.float64)
    B, L1, L2 = x.shape
    out = []
    for b in range(B):
        l1, l2 = (L1, L2) if lengths is None else (int(lengths[b][0]), int(lengths[b][1]))
        r = fn(x[b, :l1, :l2], *[None if e is None else np.asarray(e)[b, :l1, :l2]
                                  for e in extra])
        out.append((r, l1, l2))
    return out


def sw(x, gap, T, lengths=None):
    """(value [B], marginals, dS/dgap [B], dS/dT [B]) for linear SW."""
    return _first_order(lambda s, g, t: sw_value(s, g, t), x, (gap, T), lengths)


def swa(x, go, ge, T, lengths=None):
    """(value, marginals, dS/dopen, dS/dext, dS/dT) for affine SW."""
    return _first_order(lambda s, o, e, t: swa_value(s, o, e, t), x, (go, ge, T), lengths)


def nw(x, gap, T, lengths=None):
    """(value, marginals, dS/dgap, dS/dT) for linear NW."""
    return _first_order(lambda s, g, t: nw_value(s, g, t), x, (gap, T), lengths)


def dtw(x, T, bw=-1, lengths=None):
    """(value, marginals, dS/dT) for DTW."""
    return _first_order(lambda c, t: dtw_value(c, t, bw), x, (T,), lengths)


def _first_order(value_fn, x, params, lengths):
    import numpy as np
    x = np.asarray(x, dtype=np.float64)
    B, L1, L2 = x.shape
    val = np.zeros(B)
    marg = np.zeros((B, L1, L2))
    pg = np.zeros((len(params), B))
    for (r, l1, l2), b in zip(_batched(lambda e: _grads(value_fn, e, params), x, lengths),
                              range(B)):
        S, P, gp = r
        val[b] = float(S)
        marg[b, :l1, :l2] = P.numpy()
        for k, g in enumerate(gp):
            pg[k, b] = float(g)
    return (val, marg, *pg)


def hvp(family, x, V, params, lengths=None, bw=-1):
    fn = _value_fn(family, bw)
    import numpy as np
    x = np.asarray(x, dtype=np.float64)
    out = np.zeros_like(x)
    for b, (H, l1, l2) in enumerate(_batched(lambda e, v: _hvp(fn, e, params, v), x, lengths,
                                             V)):
        out[b, :l1, :l2] = H.numpy()
    return out


def param_jacobian(family, x, params, k, lengths=None, bw=-1):
    fn = _value_fn(family, bw)
    import numpy as np
    x = np.asarray(x, dtype=np.float64)
    out = np.zeros_like(x)
    for b, (J, l1, l2) in enumerate(_batched(lambda e: _param_jac(fn, e, params, k), x,
                                             lengths)):
        out[b, :l1, :l2] = J.numpy()
    return out


def _value_fn(family, bw):
    if family == "sw":
        return lambda s, g, t: sw_value(s, g, t)
    if family == "swa":
        return lambda s, o, e, t: swa_value(s, o, e, t)
    if family == "dtw":
        return lambda c, t: dtw_value(c, t, bw)
    if family == "nw":
        return lambda s, g, t: nw_value(s, g, t)
    raise ValueError(family)


# ------------------------------------------------------------------ brute force

def _paths_from(start, L1, L2, moves):
    """Every monotone path (list of (cell, move)) that starts at `start`."""
    out = []

    def rec(path):
        out.append(list(path))
        (i, j), _ = path[-1]
        for name, di, dj in moves:
            ni, nj = i + di, j + dj
            if ni < L1 and nj < L2:
                path.append(((ni, nj), name))
                rec(path)
                path.pop()

    rec([(start, "start")])
    return out


def sw_brute(s, gap, T):
    """S = T log(1 + sum over local paths exp(score / T)): a path enters at any
    cell through its score, then moves diagonally (+ score), down or right (+ gap),
    and may end at any cell it visits."""
    L1, L2 = s.shape
    moves = (("diag", 1, 1), ("down", 1, 0), ("right", 0, 1))
    total = 1.0
    for i in range(L1):
        for j in range(L2):
            for p in _paths_from((i, j), L1, L2, moves):
                sc = 0.0
                for (a, b), mv in p:
                    sc += gap if mv in ("down", "right") else float(s[a, b])
                total += math.exp(sc / T)
    return T * math.log(total)


def swa_brute(s, go, ge, T):
    """Affine gaps: a run of k down (or right) moves costs open + (k - 1) ext, a
    down run cannot turn right (or vice versa) without a diagonal move in between,
    and a path ends in any state of any visited cell."""
    L1, L2 = s.shape
    total = 1.0

    def rec(i, j, state, sc):
        nonlocal total
        total += math.exp(sc / T)
        if i + 1 < L1 and j + 1 < L2:
            rec(i + 1, j + 1, "M", sc + float(s[i + 1, j + 1]))
        if i + 1 < L1 and state in ("M", "I"):
            rec(i + 1, j, "I", sc + (go if state == "M" else ge))
        if j + 1 < L2 and state in ("M", "D"):
            rec(i, j + 1, "D", sc + (go if state == "M" else ge))

    for i in range(L1):
        for j in range(L2):
            rec(i, j, "M", float(s[i, j]))
    return T * math.log(total)


def dtw_brute(c, T):
    """S = -T log sum over monotone paths (0,0) -> (L1-1, L2-1) exp(-cost / T)."""
    L1, L2 = c.shape
    acc = 0.0

    def rec(i, j, cost):
        nonlocal acc
        if i == L1 - 1 and j == L2 - 1:
            acc += math.exp(-cost / T)
            return
        for di, dj in ((1, 1), (1, 0), (0, 1)):
            ni, nj = i + di, j + dj
            if ni < L1 and nj < L2:
                rec(ni, nj, cost + float(c[ni, nj]))

    rec(0, 0, float(c[0, 0]))
    return -T * math.log(acc)


def nw_brute(s, gap, T):
    """S = T log sum over global paths (0,0) -> (L1,L2) exp(score / T): each path
    moves diagonally (+ the score of the cell it enters), down or right (+ gap)."""
    L1, L2 = s.shape
    acc = 0.0

    def rec(i, j, sc):
        nonlocal acc
        if i == L1 and j == L2:
            acc += math.exp(sc / T)
            return
        if i < L1 and j < L2:
            rec(i + 1, j + 1, sc + float(s[i, j]))
        if i < L1:
            rec(i + 1, j, sc + gap)
        if j < L2:
            rec(i, j + 1, sc + gap)

    rec(0, 0, 0.0)
    return T * math.log(acc)
