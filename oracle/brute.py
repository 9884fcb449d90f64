"""Scalar-loop restatements of the Pairformer ops for tiny sizes (N <= 8).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

These exist to pin ``oracle.pairformer_ref`` independently of torch: every
output element is computed by explicit Python loops in float64, indexing the
pair grid by name (i, j, k) exactly as the reference's einsum strings and
softmax axes state them.  A transposed operand, a wrong einsum string, a bias
added on the wrong axis or a mask applied to the wrong index changes these
results and fails ``tests/test_oracle.py``.
"""
from __future__ import annotations

import bisect
import math

import numpy as np


def _np(t):
    return np.asarray(t.detach().double().numpy() if hasattr(t, "detach") else t, dtype=np.float64)


def _sig(x):
    return 1.0 / (1.0 + math.exp(-x))


def _ln_vec(v, w, b, eps=1e-5):
    n = len(v)
    mu = sum(v) / n
    var = sum((x - mu) ** 2 for x in v) / n
    r = 1.0 / math.sqrt(var + eps)
    return [((v[c] - mu) * r) * w[c] + b[c] for c in range(n)]


def _matvec(W, v):
    """y_o = sum_c W[o][c] v[c]  (nn.Linear convention: weight [out, in])."""
    return [sum(W[o][c] * v[c] for c in range(len(v))) for o in range(len(W))]


def layer_norm(x, w, b, eps=1e-5):
    x = _np(x); w = _np(w); b = _np(b)
    out = np.empty_like(x)
    for idx in np.ndindex(x.shape[:-1]):
        out[idx] = _ln_vec(list(x[idx]), w, b, eps)
    return out


def triangle_multiplication(z, pair_mask, W, direction):
    """z [1,N,N,C]; returns update [1,N,N,C] in float64.

    outgoing: x[i,j,d] = sum_k a[i,k,d] * b[j,k,d]
    incoming: x[i,j,d] = sum_k a[k,i,d] * b[k,j,d]
    """
    z = _np(z)[0]; m = _np(pair_mask)[0]
    W = {k: _np(v) for k, v in W.items()}
    N, _, C = z.shape
    H2 = W["p_in.weight"].shape[0]          # 2 * hidden
    Hd = H2 // 2
    xin = [[None] * N for _ in range(N)]
    a = np.zeros((N, N, Hd)); b = np.zeros((N, N, Hd))
    for i in range(N):
        for j in range(N):
            x = _ln_vec(list(z[i, j]), W["norm_in.weight"], W["norm_in.bias"])
            xin[i][j] = x
            p = _matvec(W["p_in.weight"], x)
            g = _matvec(W["g_in.weight"], x)
            y = [p[o] * _sig(g[o]) * m[i, j] for o in range(H2)]
            a[i, j] = y[:Hd]
            b[i, j] = y[Hd:]
    out = np.zeros((1, N, N, W["p_out.weight"].shape[0]))
    for i in range(N):
        for j in range(N):
            x = [0.0] * Hd
            for d in range(Hd):
                acc = 0.0
                for k in range(N):
                    if direction == "outgoing":
                        acc += a[i, k, d] * b[j, k, d]
                    else:
                        acc += a[k, i, d] * b[k, j, d]
                x[d] = acc
            xn = _ln_vec(x, W["norm_out.weight"], W["norm_out.bias"])
            po = _matvec(W["p_out.weight"], xn)
            go = _matvec(W["g_out.weight"], xin[i][j])
            out[0, i, j] = [po[o] * _sig(go[o]) for o in range(len(po))]
    return out


def triangle_attention(z, pair_mask, W, starting, n_heads, head_dim, inf=1e9, fast=False):
    """Starting node: for each row i, head h, query j:
        logit[k] = (q[i,j]/sqrt(d)) . k[i,k] + inf*(mask[i,k]-1) + bias[h][j][k],
        bias[h][j][k] = LN(z)[j,k] . Wb[h]   (shared by all rows i)
    Ending node: the same on z^T / mask^T, output transposed back.
    ``fast``: the rows of W_q, W_k, W_v, W_g, the vectors q, k, v, g (before the sigmoid)
    and the output vector pass through mx8_vec.
    """
    z = _np(z)[0]; m = _np(pair_mask)[0]
    W = {k: _np(v) for k, v in W.items()}
    fq = mx8_vec if fast else (lambda vec: vec)
    if fast:
        for key in ("mha.linear_q.weight", "mha.linear_k.weight", "mha.linear_v.weight", "mha.linear_g.weight"):
            W[key] = np.array([mx8_vec(list(r)) for r in W[key]])
    if not starting:
        z = z.transpose(1, 0, 2); m = m.T
    N = z.shape[0]
    H, D = n_heads, head_dim
    x = [[_ln_vec(list(z[i, j]), W["layer_norm.weight"], W["layer_norm.bias"]) for j in range(N)]
         for i in range(N)]
    bias = [[[sum(x[j][kk][c] * W["linear.weight"][h][c] for c in range(len(x[j][kk])))
              for kk in range(N)] for j in range(N)] for h in range(H)]
    q = [[fq(_matvec(W["mha.linear_q.weight"], x[i][j])) for j in range(N)] for i in range(N)]
    k = [[fq(_matvec(W["mha.linear_k.weight"], x[i][j])) for j in range(N)] for i in range(N)]
    v = [[fq(_matvec(W["mha.linear_v.weight"], x[i][j])) for j in range(N)] for i in range(N)]
    g = [[[_sig(t) for t in fq(_matvec(W["mha.linear_g.weight"], x[i][j]))] for j in range(N)]
         for i in range(N)]
    out = np.zeros((1, N, N, W["mha.linear_o.weight"].shape[0]))
    for i in range(N):
        for j in range(N):
            o = [0.0] * (H * D)
            for h in range(H):
                logits = []
                for kk in range(N):
                    dot = sum((q[i][j][h * D + d] / math.sqrt(D)) * k[i][kk][h * D + d]
                              for d in range(D))
                    # the reference adds in fp32, mask term first (boltz2.py:802-803):
                    # at |x| ~ 1e9 the fp32 sum swallows the O(1) terms, which makes a
                    # fully masked row uniform.  Reproduce those two roundings.
                    f32 = np.float32
                    lg = f32(f32(dot) + f32(inf * (m[i, kk] - 1.0)))
                    logits.append(float(f32(lg + f32(bias[h][j][kk]))))
                mx = max(logits)
                e = [math.exp(t - mx) for t in logits]
                s = sum(e)
                for d in range(D):
                    o[h * D + d] = sum(e[kk] / s * v[i][kk][h * D + d] for kk in range(N))
            o = [o[c] * g[i][j][c] for c in range(H * D)]
            out[0, i, j] = fq(_matvec(W["mha.linear_o.weight"], o))
    if not starting:
        out = out.transpose(0, 2, 1, 3)
    return out


def transition(x, W):
    x = _np(x)
    W = {k: _np(v) for k, v in W.items()}
    out = np.zeros(x.shape[:-1] + (W["fc3.weight"].shape[0],))
    for idx in np.ndindex(x.shape[:-1]):
        xn = _ln_vec(list(x[idx]), W["norm.weight"], W["norm.bias"])
        h1 = _matvec(W["fc1.weight"], xn)
        h2 = _matvec(W["fc2.weight"], xn)
        hh = [h1[t] * _sig(h1[t]) * h2[t] for t in range(len(h1))]
        out[idx] = _matvec(W["fc3.weight"], hh)
    return out


def attention_pair_bias(s, z, mask, k_in, W, num_heads, inf=1e6, fast=False):
    """out_i = proj_o( sigmoid(proj_g s_i) * concat_h sum_j p_hij v_jh ),
    p_hij = softmax_j( q_ih . k_jh / sqrt(d) + LN(z_ij) . Wz[h] - inf*(1-mask_j) ).
    ``fast``: the gated vector passes through mx8_vec before proj_o.
    """
    s = _np(s)[0]; z = _np(z)[0]; mask = _np(mask)[0]; k_in = _np(k_in)[0]
    W = {k: _np(v) for k, v in W.items()}
    N, C = s.shape
    H = num_heads; D = C // H
    q = [[a + bb for a, bb in zip(_matvec(W["proj_q.weight"], s[i]), W["proj_q.bias"])]
         for i in range(N)]
    kk = [_matvec(W["proj_k.weight"], k_in[j]) for j in range(N)]
    vv = [_matvec(W["proj_v.weight"], k_in[j]) for j in range(N)]
    g = [[_sig(t) for t in _matvec(W["proj_g.weight"], s[i])] for i in range(N)]
    zb = [[_matvec(W["proj_z.1.weight"], _ln_vec(list(z[i, j]), W["proj_z.0.weight"],
                                                 W["proj_z.0.bias"])) for j in range(N)]
          for i in range(N)]
    out = np.zeros((1, N, C))
    for i in range(N):
        o = [0.0] * C
        for h in range(H):
            logits = [sum(q[i][h * D + d] * kk[j][h * D + d] for d in range(D)) / math.sqrt(D)
                      + zb[i][j][h] + (1.0 - mask[j]) * -inf for j in range(N)]
            mx = max(logits)
            e = [math.exp(t - mx) for t in logits]
            ssum = sum(e)
            for d in range(D):
                o[h * D + d] = sum(e[j] / ssum * vv[j][h * D + d] for j in range(N))
        go = [g[i][c] * o[c] for c in range(C)]
        out[0, i] = _matvec(W["proj_o.weight"], mx8_vec(go) if fast else go)
    return out


def pairformer_layer(s, z, mask, pair_mask, W, tri_heads, tri_dim, att_heads):
    """Layer composed from the scalar ops above, in ``reference.py:877-912`` order."""
    def sub(p):
        return {k[len(p) + 1:]: v for k, v in W.items() if k.startswith(p + ".")}
    z = _np(z)
    z = z + triangle_multiplication(z, pair_mask, sub("tri_mul_out"), "outgoing")
    z = z + triangle_multiplication(z, pair_mask, sub("tri_mul_in"), "incoming")
    z = z + triangle_attention(z, pair_mask, sub("tri_att_start"), True, tri_heads, tri_dim)
    z = z + triangle_attention(z, pair_mask, sub("tri_att_end"), False, tri_heads, tri_dim)
    z = z + transition(z, sub("transition_z"))
    if s is None:
        return None, z
    s = _np(s)
    sn = layer_norm(s, W["pre_norm_s.weight"], W["pre_norm_s.bias"])
    s = s + attention_pair_bias(sn, z, mask, sn, sub("attention"), att_heads)
    s = s + transition(s, sub("transition_s"))
    return s, z


# --------------------------------------------------------------------------------------
# MXFP8 (fast mode) by scalar loops: the quantizer below shares no code with fp8_emu.
# Element rounding searches the e4m3 code table for the nearest value (ties to the even
# code); the block exponent comes from math.frexp.
# --------------------------------------------------------------------------------------
def _e4m3_value(code):
    s, e, m = code >> 7, (code >> 3) & 15, code & 7
    v = m * 2.0 ** -9 if e == 0 else (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return -v if s else v


_E4M3_POS = sorted((_e4m3_value(c), c) for c in range(0x7F))    # non-negative finite codes
_E4M3_VALS = [v for v, _ in _E4M3_POS]


def _e4m3_nearest(v):
    """Nearest e4m3 value to v (|v| clamped to 448), ties to the even code: a table search
    between the two neighbouring code values."""
    a = min(abs(v), 448.0)
    hi = bisect.bisect_left(_E4M3_VALS, a)
    if hi == 0:
        q = _E4M3_VALS[0]
    elif hi == len(_E4M3_VALS):
        q = _E4M3_VALS[-1]
    else:
        (lv, lc), (hv, hc) = _E4M3_POS[hi - 1], _E4M3_POS[hi]
        dl, dh = a - lv, hv - a
        q = lv if (dl < dh or (dl == dh and lc % 2 == 0)) else hv
    return -q if v < 0 else q


def mx8_block(vals):
    """Quantize-dequantize one block of 32 values with the smallest power of two X such
    that amax / X <= 448, found by walking the exponent up from amax's."""
    amax = max(abs(v) for v in vals)
    if amax == 0.0:
        return [0.0] * len(vals)
    _, ex = math.frexp(amax)            # amax = f * 2^ex, 0.5 <= f < 1
    e = ex - 12                         # amax / 2^e = f * 4096 >= 2048 > 448: too small
    while amax / 2.0 ** e > 448.0:
        e += 1
    X = 2.0 ** e
    return [_e4m3_nearest(v / X) * X for v in vals]


def mx8_vec(v):
    out = []
    for b0 in range(0, len(v), 32):
        out += mx8_block(list(v[b0:b0 + 32]))
    return out


def _matvec_mx8(Wq, v):
    """Both operands quantized along the input axis (Wq rows already quantized)."""
    vq = mx8_vec(v)
    return [sum(Wq[o][c] * vq[c] for c in range(len(vq))) for o in range(len(Wq))]


def triangle_multiplication_mx8(z, pair_mask, W, direction):
    """Fast-mode triangle multiplication; quantization points as in
    ``pairformer_ref.triangle_multiplication_mx8``."""
    z = _np(z)[0]; m = _np(pair_mask)[0]
    W = {k: _np(v) for k, v in W.items()}
    Wq = {k: [mx8_vec(list(r)) for r in W[k]] for k in ("p_in.weight", "g_in.weight", "p_out.weight",
                                                          "g_out.weight")}
    N, _, C = z.shape
    Hd = W["p_in.weight"].shape[0] // 2
    xin = [[None] * N for _ in range(N)]
    a = np.zeros((N, N, Hd)); b = np.zeros((N, N, Hd))
    for i in range(N):
        for j in range(N):
            x = _ln_vec(list(z[i, j]), W["norm_in.weight"], W["norm_in.bias"])
            xin[i][j] = x
            p = _matvec_mx8(Wq["p_in.weight"], x)
            g = _matvec_mx8(Wq["g_in.weight"], x)
            y = [p[o] * _sig(g[o]) * m[i, j] for o in range(2 * Hd)]
            a[i, j] = y[:Hd]
            b[i, j] = y[Hd:]
    # quantize a, b along the contraction index k
    aq = np.zeros_like(a); bq = np.zeros_like(b)
    for d in range(Hd):
        for r in range(N):
            if direction == "outgoing":      # k = second index
                aq[r, :, d] = mx8_vec(list(a[r, :, d])); bq[r, :, d] = mx8_vec(list(b[r, :, d]))
            else:                            # k = first index
                aq[:, r, d] = mx8_vec(list(a[:, r, d])); bq[:, r, d] = mx8_vec(list(b[:, r, d]))
    out = np.zeros((1, N, N, W["p_out.weight"].shape[0]))
    for i in range(N):
        for j in range(N):
            x = [0.0] * Hd
            for d in range(Hd):
                acc = 0.0
                for k in range(N):
                    if direction == "outgoing":
                        acc += aq[i, k, d] * bq[j, k, d]
                    else:
                        acc += aq[k, i, d] * bq[k, j, d]
                x[d] = acc
            xn = _ln_vec(x, W["norm_out.weight"], W["norm_out.bias"])
            po = _matvec_mx8(Wq["p_out.weight"], xn)
            go = _matvec_mx8(Wq["g_out.weight"], xin[i][j])
            out[0, i, j] = [po[o] * _sig(go[o]) for o in range(len(po))]
    return out


def transition_mx8(x, W):
    x = _np(x)
    W = {k: _np(v) for k, v in W.items()}
    Wq = {k: [mx8_vec(list(r)) for r in W[k]] for k in ("fc1.weight", "fc2.weight", "fc3.weight")}
    out = np.zeros(x.shape[:-1] + (W["fc3.weight"].shape[0],))
    for idx in np.ndindex(x.shape[:-1]):
        xn = _ln_vec(list(x[idx]), W["norm.weight"], W["norm.bias"])
        h1 = _matvec_mx8(Wq["fc1.weight"], xn)
        h2 = _matvec_mx8(Wq["fc2.weight"], xn)
        hh = [h1[t] * _sig(h1[t]) * h2[t] for t in range(len(h1))]
        out[idx] = _matvec_mx8(Wq["fc3.weight"], hh)
    return out


# ----------------------------------------------------------------------------- MSA module
def outer_product_mean(m, msa_mask, W):
    """z[b,i,j,o] = sum_k Wo[o][k] f[k] + bo[o], f[c*H + d] = sum_s a[s,i,c] b[s,j,d] / n_ij,
    n_ij = max(1, sum_s mask[s,i] mask[s,j]); a, b = proj(LN(m[s,i])) * mask[s,i]."""
    m, msk = _np(m), _np(msa_mask)
    W = {k: _np(v) for k, v in W.items()}
    B, S, N, _ = m.shape
    Hh = W["proj_a.weight"].shape[0]
    a = np.zeros((B, S, N, Hh))
    b = np.zeros((B, S, N, Hh))
    for bb in range(B):
        for s in range(S):
            for i in range(N):
                xn = _ln_vec(list(m[bb, s, i]), W["norm.weight"], W["norm.bias"])
                a[bb, s, i] = np.array(_matvec(W["proj_a.weight"], xn)) * msk[bb, s, i]
                b[bb, s, i] = np.array(_matvec(W["proj_b.weight"], xn)) * msk[bb, s, i]
    out = np.zeros((B, N, N, W["proj_o.weight"].shape[0]))
    for bb in range(B):
        for i in range(N):
            for j in range(N):
                n = max(1.0, sum(msk[bb, s, i] * msk[bb, s, j] for s in range(S)))
                f = [sum(a[bb, s, i, c] * b[bb, s, j, d] for s in range(S)) / n
                     for c in range(Hh) for d in range(Hh)]
                out[bb, i, j] = np.array(_matvec(W["proj_o.weight"], f)) + W["proj_o.bias"]
    return out


def pair_weighted_averaging(m, z, pair_mask, W, num_heads, c_h, inf=1e6):
    """o[s,i,h*c_h+d] = sigmoid(g[s,i,h,d]) * sum_j w[h,i,j] v[s,j,h,d], w = softmax over j
    of (LN(z[i,j]) . Wz[h]) - inf*(1 - mask[i,j]); out = proj_o(o)."""
    m, z, pm = _np(m), _np(z), _np(pair_mask)
    W = {k: _np(v) for k, v in W.items()}
    B, S, N, _ = m.shape
    out = np.zeros((B, S, N, W["proj_o.weight"].shape[0]))
    for bb in range(B):
        mn = {(s, i): _ln_vec(list(m[bb, s, i]), W["norm_m.weight"], W["norm_m.bias"])
              for s in range(S) for i in range(N)}
        v = {k: _matvec(W["proj_m.weight"], x) for k, x in mn.items()}
        g = {k: [_sig(t) for t in _matvec(W["proj_g.weight"], x)] for k, x in mn.items()}
        logit = {}
        for i in range(N):
            for j in range(N):
                zn = _ln_vec(list(z[bb, i, j]), W["norm_z.weight"], W["norm_z.bias"])
                lg = _matvec(W["proj_z.weight"], zn)
                for h in range(num_heads):
                    logit[h, i, j] = lg[h] - inf * (1.0 - pm[bb, i, j])
        wts = {}
        for h in range(num_heads):
            for i in range(N):
                mx = max(logit[h, i, j] for j in range(N))
                e = [math.exp(logit[h, i, j] - mx) for j in range(N)]
                den = sum(e)
                for j in range(N):
                    wts[h, i, j] = e[j] / den
        for s in range(S):
            for i in range(N):
                o = [g[s, i][h * c_h + d] * sum(wts[h, i, j] * v[s, j][h * c_h + d] for j in range(N))
                     for h in range(num_heads) for d in range(c_h)]
                out[bb, s, i] = _matvec(W["proj_o.weight"], o)
    return out


def pairwise_conditioning(z_trunk, rel_pos, W, n_transitions=2):
    """PairwiseConditioning (boltz2.py:1344-1355) by loops: per pair, LN over the 2c
    concatenated channels, the 2c -> c projection, then x += transition_i(x)."""
    zt = _np(z_trunk); rp = _np(rel_pos)
    W = {k: _np(v) for k, v in W.items()}
    out = np.zeros(zt.shape)
    for idx in np.ndindex(zt.shape[:-1]):
        v = list(zt[idx]) + list(rp[idx])
        x = _matvec(W["dim_pairwise_init_proj.1.weight"],
                    _ln_vec(v, W["dim_pairwise_init_proj.0.weight"], W["dim_pairwise_init_proj.0.bias"]))
        for i in range(n_transitions):
            p = f"transitions.{i}."
            xn = _ln_vec(x, W[p + "norm.weight"], W[p + "norm.bias"])
            h1 = _matvec(W[p + "fc1.weight"], xn)
            h2 = _matvec(W[p + "fc2.weight"], xn)
            hh = [h1[t] * _sig(h1[t]) * h2[t] for t in range(len(h1))]
            y = _matvec(W[p + "fc3.weight"], hh)
            x = [x[c] + y[c] for c in range(len(x))]
        out[idx] = x
    return out


def token_trans_bias(z, W, depth):
    """DiffusionConditioning's token_trans_bias (boltz2.py:2472-2475) by loops: output
    index l * H + h is layer l's LN (its own affine) followed by its head-h weight row."""
    z = _np(z)
    W = {k: _np(v) for k, v in W.items()}
    H = W["token_trans_proj_z.0.1.weight"].shape[0]
    out = np.zeros(z.shape[:-1] + (depth * H,))
    for idx in np.ndindex(z.shape[:-1]):
        for l in range(depth):
            p = f"token_trans_proj_z.{l}."
            xn = _ln_vec(list(z[idx]), W[p + "0.weight"], W[p + "0.bias"])
            y = _matvec(W[p + "1.weight"], xn)
            for h in range(H):
                out[idx + (l * H + h,)] = y[h]
    return out
