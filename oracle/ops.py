"""Plain-PyTorch CPU restatement of the reference kernels (test infrastructure).

Reference = SkyeGunasekaran/fastAlgebraicTransformer, files as they appear in
the reference checkout (fused_ops.py, forward.py, backward.py, tests.py,
algebraic_model.py). Each function states the lines it restates.
"""

import math

import torch

# fused_ops.py:20 -- EPS = 1e-6 ; fused_ops.py:21 / tests.py:59 -- masked fill value
EPS = 1e-6
NEG_FILL = -1e4


def _up(t, dtype):
    return t.detach().to(device="cpu", dtype=dtype)


# ---------------------------------------------------------------------------
# rational sigmoid -- fused_ops.py:28-45 (and inlined at fused_ops.py:81-82,
# forward.py:137-138, backward.py:137-139); tests.py:20-22
# ---------------------------------------------------------------------------

def rsig(x):
    """sigma(x) = 0.5 * (x / (|x| + 1) + 1)  (fused_ops.py:34-35)."""
    return 0.5 * (x / (x.abs() + 1.0) + 1.0)


def rsig_deriv(x):
    """sigma'(x) = 0.5 / (|x| + 1)^2  (fused_ops.py:43-45)."""
    d = x.abs() + 1.0
    return 0.5 / (d * d)


def _sig4(x):
    # fused_ops.py:85-86: sigma2 = sigma*sigma ; sigma4 = sigma2*sigma2
    s = rsig(x)
    s2 = s * s
    return s2 * s2


# ---------------------------------------------------------------------------
# rational softmax -- fwd fused_ops.py:52-106 (CPU path :611-615, tests.py:25-29)
#                     bwd fused_ops.py:150-189
# ---------------------------------------------------------------------------

def rational_softmax_fwd(x, eps=EPS, dtype=torch.float64):
    """p = sigma(x)^4 / (sum_row sigma(x)^4 + eps) over the last dim."""
    x = _up(x, dtype)
    f = _sig4(x)
    return f / (f.sum(dim=-1, keepdim=True) + eps)


def rational_softmax_bwd(dy, x, p, eps=EPS, dtype=torch.float64):
    """dx = p * g * (dy - <dy, p>),  g = 2 / ((|x|+1)^2 (sigma + eps)).

    Follows the kernel (fused_ops.py:157-187), which uses the *saved* p and
    puts eps next to sigma in g (fused_ops.py:184)."""
    dy, x, p = _up(dy, dtype), _up(x, dtype), _up(p, dtype)
    dot = (dy * p).sum(dim=-1, keepdim=True)
    den = x.abs() + 1.0
    sig = 0.5 * (x / den + 1.0)
    g = 2.0 / (den * den * (sig + eps))
    return p * g * (dy - dot)


# ---------------------------------------------------------------------------
# rational SwiGLU -- fwd fused_ops.py:196-229 (CPU :624-626, tests.py:32-35)
#                    bwd fused_ops.py:236-288
# ---------------------------------------------------------------------------

def swiglu_fwd(gate, value, dtype=torch.float64):
    """out = gate * sigma(gate) * value  (fused_ops.py:223-227)."""
    g, v = _up(gate, dtype), _up(value, dtype)
    return g * rsig(g) * v


def swiglu_bwd(dy, gate, value, dtype=torch.float64):
    """dvalue = dy*gate*sigma ; dgate = dy*value*(sigma + gate*sigma')
    (fused_ops.py:276-285). Returns (dgate, dvalue)."""
    dy, g, v = _up(dy, dtype), _up(gate, dtype), _up(value, dtype)
    den = g.abs() + 1.0
    sig = 0.5 * (g / den + 1.0)
    sd = 0.5 / (den * den)
    return dy * v * (sig + g * sd), dy * g * sig


# ---------------------------------------------------------------------------
# mean-error norm -- fwd fused_ops.py:295-342 (CPU :635-636, tests.py:38-41)
#                    bwd fused_ops.py:349-423 + torch dgamma :593-597
# ---------------------------------------------------------------------------

def mean_error_norm_fwd(x, weight, eps=EPS, dtype=torch.float64):
    """Returns (y, mu): mu = mean|x| per row, stored WITHOUT eps
    (fused_ops.py:326,330); y = x / (mu + eps) * weight (fused_ops.py:327,340)."""
    x, w = _up(x, dtype), _up(weight, dtype)
    mu = x.abs().mean(dim=-1)
    y = x / (mu.unsqueeze(-1) + eps) * w
    return y, mu


def mean_error_norm_bwd(dy, x, weight, mu, eps=EPS, dtype=torch.float64):
    """Returns (dx, dweight).

    dx = dy*w/mu' - sign(x) * (sum(dy*y)/n) / mu',  mu' = mu + eps
    (fused_ops.py:389-421). dweight = sum over rows of dy * x / mu'
    (fused_ops.py:595-597). sign follows torch's abs backward, sign(0) = 0;
    the reference Triton kernel uses +1 at exactly zero (fused_ops.py:418),
    a case that random inputs never produce."""
    dy, x, w, mu = _up(dy, dtype), _up(x, dtype), _up(weight, dtype), _up(mu, dtype)
    n = x.shape[-1]
    inv = 1.0 / (mu.unsqueeze(-1) + eps)
    y = x * inv * w
    c = (dy * y).sum(dim=-1, keepdim=True)
    dx = dy * w * inv - torch.sign(x) * (c / n) * inv
    dw = (dy * (x * inv)).reshape(-1, n).sum(dim=0)
    return dx, dw


# ---------------------------------------------------------------------------
# ALiBi slopes -- forward.py:21-42
# ---------------------------------------------------------------------------

def alibi_slopes(n_heads):
    """slopes[i] = b^(i+1), b = 2^(-8/p), p = largest power of two <= n;
    the n - p extra heads take the odd powers of 2^(-8/(2p)). Powers are taken
    with torch.pow on a float base and int64 exponents (float32 result), the
    arithmetic route of forward.py:30-31,36."""
    p = 2 ** int(math.floor(math.log2(n_heads)))
    out = torch.pow(2.0 ** (-8.0 / p), torch.arange(1, p + 1))
    if p != n_heads:
        rem = min(p, n_heads - p)
        out = torch.cat([out, torch.pow(2.0 ** (-8.0 / (2 * p)), torch.arange(1, 2 * rem, 2))])
    return out.to(torch.float32)


# ---------------------------------------------------------------------------
# rational attention -- fwd forward.py:49-159 ; bwd backward.py:62-266
# Layout [B, H, T, D]. The reference kernels are always causal
# (forward.py:110, backward.py:125,222). Two extensions, following the
# reference model's CPU attention (algebraic_model.py:112-136): a key padding
# mask [B, T] (key j of batch b is dropped where mask[b, j] == 0,
# algebraic_model.py:129-131) and a non-causal mode (every key visible, ALiBi
# -slope * |i - j| as that CPU path writes it, algebraic_model.py:118-121).
# Dropped keys contribute exactly nothing here (the reference CPU path's -1e4
# fill leaves sigma(-1e4)^4 ~ 6e-18 per key).
# ---------------------------------------------------------------------------

def _scores(q, k, slopes, scale, causal=True, key_mask=None):
    # forward.py:129-133: s = (q.k) * scale - slope * |i - j|
    T = q.shape[-2]
    s = torch.matmul(q, k.transpose(-1, -2)) * scale
    pos = torch.arange(T)
    dist = (pos[:, None] - pos[None, :]).abs().to(q.dtype)
    s = s - slopes.to(q.dtype).view(1, -1, 1, 1) * dist
    keep = (pos[None, :] <= pos[:, None]) if causal else torch.ones(T, T, dtype=torch.bool)
    keep = keep[None, None]
    if key_mask is not None:
        keep = keep & (key_mask.to("cpu") != 0)[:, None, None, :]
    return s, keep


def _chunks(B, H, chunk):
    if chunk is None:
        yield slice(None), slice(None)
        return
    for b in range(B):
        for h0 in range(0, H, chunk):
            yield slice(b, b + 1), slice(h0, min(H, h0 + chunk))


def _mask_rows(key_mask, bs):
    return None if key_mask is None else key_mask[bs]


def attention_fwd(q, k, v, slopes, scale, eps=EPS, dtype=torch.float64, chunk=None,
                  causal=True, key_mask=None):
    """Returns (o, L). f = sigma(s)^4 for j <= i only (the kernel never visits
    j > i, forward.py:110,119); L = sum f stored WITHOUT eps (forward.py:159);
    o = sum f v / (L + eps) (forward.py:150-151). ``chunk`` bounds memory by
    processing ``chunk`` heads of one batch entry at a time (heads are
    independent). ``causal=False`` / ``key_mask``: the extensions above."""
    q, k, v = _up(q, dtype), _up(k, dtype), _up(v, dtype)
    slopes = _up(slopes, dtype)
    B, H, T, D = q.shape
    o = torch.empty_like(q)
    L = torch.empty(B, H, T, dtype=dtype)
    for bs, hs in _chunks(B, H, chunk):
        s, keep = _scores(q[bs, hs], k[bs, hs], slopes[hs], scale, causal,
                          _mask_rows(key_mask, bs))
        f = torch.where(keep, _sig4(s), torch.zeros((), dtype=dtype))
        l = f.sum(dim=-1)
        L[bs, hs] = l
        o[bs, hs] = torch.matmul(f, v[bs, hs]) / (l + eps).unsqueeze(-1)
    return o, L


def attention_delta(o, do, dtype=torch.float64):
    """Delta_i = <dO_i, O_i> (backward.py:117, recomputed per pair at :248)."""
    return (_up(o, dtype) * _up(do, dtype)).sum(dim=-1)


def attention_bwd(q, k, v, o, L, do, slopes, scale, eps=EPS, dtype=torch.float64,
                  chunk=None, causal=True, key_mask=None):
    """Returns (dq, dk, dv) following backward.py:116-154 (dQ) and
    backward.py:232-260 (dK, dV):
      p = f / (L + eps),  g = 2 / ((|s|+1)^2 (sigma + eps)),
      dS = p * g * (dO.v - Delta),  dQ = scale dS K,  dK = scale dS^T Q,
      dV = P^T dO ;  only pairs j <= i contribute (with ``causal=False`` every
    pair; with ``key_mask`` only unmasked keys)."""
    q, k, v, o, do = (_up(t, dtype) for t in (q, k, v, o, do))
    L = _up(L, dtype)
    slopes = _up(slopes, dtype)
    B, H, T, D = q.shape
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    for bs, hs in _chunks(B, H, chunk):
        qq, kk, vv, oo, dd = q[bs, hs], k[bs, hs], v[bs, hs], o[bs, hs], do[bs, hs]
        s, keep = _scores(qq, kk, slopes[hs], scale, causal, _mask_rows(key_mask, bs))
        den = s.abs() + 1.0
        sig = 0.5 * (s / den + 1.0)
        s2 = sig * sig
        f = s2 * s2
        p = f / (L[bs, hs] + eps).unsqueeze(-1)
        g = 2.0 / (den * den * (sig + eps))
        delta = (dd * oo).sum(dim=-1, keepdim=True)
        dp = torch.matmul(dd, vv.transpose(-1, -2))
        zero = torch.zeros((), dtype=dtype)
        ds = torch.where(keep, p * g * (dp - delta), zero)
        p = torch.where(keep, p, zero)
        dq[bs, hs] = torch.matmul(ds, kk) * scale
        dk[bs, hs] = torch.matmul(ds.transpose(-1, -2), qq) * scale
        dv[bs, hs] = torch.matmul(p.transpose(-1, -2), dd)
    return dq, dk, dv


def harness_attention(q, k, v, slopes, scale, eps=EPS, causal=True, key_mask=None):
    """The reference test harness formulation (tests.py:44-65 and the model's
    CPU path algebraic_model.py:112-136): full score matrix, ALiBi, the -1e4
    causal fill, the -1e4 padding fill where key_mask == 0
    (algebraic_model.py:129-131), rational softmax over all T columns, then
    P @ V. ``causal=False`` drops the causal fill. Pure torch ops on whatever
    dtype/grad state the inputs carry (used with autograd)."""
    B, H, T, D = q.shape
    scores = torch.matmul(q, k.transpose(-2, -1)) * scale
    pos = torch.arange(T)
    rel = pos[:, None] - pos[None, :]
    scores = scores + (-rel.abs().to(q.dtype) * slopes.to(q.dtype).view(1, H, 1, 1))
    if causal:
        upper = torch.triu(torch.ones(T, T, dtype=torch.bool), diagonal=1)
        scores = scores.masked_fill(upper[None, None], NEG_FILL)
    if key_mask is not None:
        pad = key_mask.to("cpu")[:, None, None, :] == 0
        scores = scores.masked_fill(pad, NEG_FILL)
    sig = 0.5 * (scores / (scores.abs() + 1.0) + 1.0)
    f = sig.pow(4)
    probs = f / (f.sum(dim=-1, keepdim=True) + eps)
    return torch.matmul(probs, v)


def loop_attention_fwd(q, k, v, slopes, scale, eps=EPS, causal=True, key_mask=None):
    """Scalar pure-Python loop over (b, h, i, j <= i), as the reference kernel
    walks it (forward.py:80-159); ``causal=False`` walks every j, ``key_mask``
    skips masked keys. Only for tiny inputs."""
    q, k, v = (_up(t, torch.float64).tolist() for t in (q, k, v))
    sl = _up(slopes, torch.float64).tolist()
    B, H, T, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    km = None if key_mask is None else key_mask.to("cpu").tolist()
    o = [[[[0.0] * D for _ in range(T)] for _ in range(H)] for _ in range(B)]
    L = [[[0.0] * T for _ in range(H)] for _ in range(B)]
    for b in range(B):
        for h in range(H):
            for i in range(T):
                acc = [0.0] * D
                l = 0.0
                for j in range(i + 1 if causal else T):
                    if km is not None and km[b][j] == 0:
                        continue
                    s = sum(q[b][h][i][d] * k[b][h][j][d] for d in range(D)) * scale
                    s = s - sl[h] * abs(i - j)
                    sig = 0.5 * (s / (abs(s) + 1.0) + 1.0)
                    f = (sig * sig) * (sig * sig)
                    l += f
                    for d in range(D):
                        acc[d] += f * v[b][h][j][d]
                inv = 1.0 / (l + eps)
                o[b][h][i] = [a * inv for a in acc]
                L[b][h][i] = l
    return torch.tensor(o, dtype=torch.float64), torch.tensor(L, dtype=torch.float64)
