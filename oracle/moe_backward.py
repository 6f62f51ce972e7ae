"""fp64 restatement of the MoE layer's backward pass and load-balancing loss
(test infrastructure, not shipped).

The reference has no backward for the FFN/MoE half (its block backward,
src/transformer.c:975-1013, skips it) and no code for the auxiliary loss
its moe_forward comment defines (src/transformer.c:280-282):
    aux = n_experts * sum_e f_e * P_e,
here with f_e = (assignments to e) / (T * k) (a count, no gradient) and
P_e = mean_t probs[t, e].  The layer (src/transformer.c:287-366) is
    probs = softmax(x W_r), top-k ids, gw = p_sel / sum p_sel,
    out[t] = sum_slots gw * (silu(x W_g) * (x W_u)) W_d   (per expert),
and the loss differentiated is L = sum(dout * out) + aux_coef * aux, with the
routing decisions (ids) held fixed as the forward made them.  Everything is
float64; moe_forward64 is the matching forward, so finite differences of it
pin moe_backward64 (tests/test_backward.py).
"""
import numpy as np


def _silu(g):
    return g / (1.0 + np.exp(-g))


def moe_forward64(x, wr, wg, wu, wd, ids, bias=None):
    """out [T x d] and probs [T x E] in float64 for fixed expert ids [T x k].
    wg, wu: [E][d x F], wd: [E][F x d], wr: [d x E]."""
    x = np.asarray(x, np.float64)
    logits = x @ wr
    if bias is not None:
        logits = logits + bias
    z = logits - logits.max(axis=1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(axis=1, keepdims=True)
    T, k = ids.shape
    psel = np.take_along_axis(p, ids, axis=1)
    gw = psel / psel.sum(axis=1, keepdims=True)
    out = np.zeros_like(x)
    for t in range(T):
        for s in range(k):
            e = ids[t, s]
            h = _silu(x[t] @ wg[e]) * (x[t] @ wu[e])
            out[t] += gw[t, s] * (h @ wd[e])
    return out, p


def aux_loss64(p, ids, E):
    T, k = ids.shape
    f = np.bincount(ids.ravel(), minlength=E) / float(T * k)
    return E * float(np.sum(f * p.mean(axis=0))), f


def moe_backward64(x, wr, wg, wu, wd, ids, dout, aux_coef=0.0, bias=None):
    """Gradients of L = sum(dout * out) + aux_coef * aux: dict with dx,
    dwr, dwg, dwu, dwd (shapes of x, wr, wg, wu, wd) and the loss terms."""
    x = np.asarray(x, np.float64)
    dout = np.asarray(dout, np.float64)
    wr, wg, wu, wd = (np.asarray(a, np.float64) for a in (wr, wg, wu, wd))
    T, d = x.shape
    E = wr.shape[1]
    k = ids.shape[1]
    out, p = moe_forward64(x, wr, wg, wu, wd, ids, bias)
    psel = np.take_along_axis(p, ids, axis=1)
    S = psel.sum(axis=1, keepdims=True)
    gw = psel / S
    dx = np.zeros_like(x)
    dwg, dwu, dwd = np.zeros_like(wg), np.zeros_like(wu), np.zeros_like(wd)
    dgw = np.zeros((T, k))
    for t in range(T):
        for s in range(k):
            e = ids[t, s]
            g, u = x[t] @ wg[e], x[t] @ wu[e]
            sg = 1.0 / (1.0 + np.exp(-g))
            h = g * sg * u
            y = h @ wd[e]
            dgw[t, s] = dout[t] @ y
            dy = gw[t, s] * dout[t]
            dwd[e] += np.outer(h, dy)
            dh = wd[e] @ dy
            dg = dh * u * (sg + g * sg * (1.0 - sg))
            du = dh * g * sg
            dwg[e] += np.outer(x[t], dg)
            dwu[e] += np.outer(x[t], du)
            dx[t] += wg[e] @ dg + wu[e] @ du
    # gw = p_sel / S  ->  d p_sel
    dpsel = dgw / S - (dgw * gw).sum(axis=1, keepdims=True) / S
    dp = np.zeros_like(p)
    np.put_along_axis(dp, ids, dpsel, axis=1)
    aux, f = aux_loss64(p, ids, E)
    dp += aux_coef * E * f[None, :] / T
    dlogits = p * (dp - (dp * p).sum(axis=1, keepdims=True))
    dwr = x.T @ dlogits
    dx += dlogits @ wr.T
    return dict(dx=dx, dwr=dwr, dwg=dwg, dwu=dwu, dwd=dwd, out=out, probs=p, aux=aux,
                loss=float(np.sum(dout * out)) + aux_coef * aux, dlogits=dlogits)
