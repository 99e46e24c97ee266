"""CPU oracle for the DeepSeek-V3 / Kimi-K2 MLA attention layer around the MLA kernels.

TEST INFRASTRUCTURE ONLY. This module is the checker: only ``tests/`` may import it. The
product layer (``minisgl_amd.layers``) never calls it.

The reference has no MLA layer (its only attention caller is the MHA ``AttentionLayer``,
python/minisgl/layers/attention.py:17-57; ``models/register.py:5-12`` lists no DeepSeek or
Kimi model), so this restates the published DeepSeek-V2/V3 MLA layer -- the ``DeepseekV3Attention``
module of the DeepSeek-V3 release (HF ``modeling_deepseek.py``, not vendored here) -- in its
decompressed (non-absorbed) form, over a request's whole token history, with no paging:

* ``q = W_qb rmsnorm(W_qa x)``, split per head into 128 nope + 64 rope dims;
* ``[c | k_pe] = W_kva x``; ``c = rmsnorm(c)``; ``k_pe`` is one 64-dim rope key per token,
  shared by all heads;
* ``W_kvb`` viewed ``[H, 128 + 128, 512]``: its first 128 rows per head give ``k_nope = W_UK c``,
  the last 128 ``v = W_UV c`` (the split of ``kv_b_proj``'s output in that module);
* RoPE on ``q_pe`` and ``k_pe`` with angle ``position * inv_freq[i]`` computed here in float64
  (not through a cos/sin cache); ``inv_freq = base^(-2i/d)``, blended for YaRN as
  python/minisgl/layers/rotary.py:92-111 does; interleaved pairs ``(2i, 2i+1)`` (DeepSeek's
  layout) or halves ``(i, i + d/2)`` (rotary.py's flashinfer call, which rotates halves);
  YaRN's cos/sin amplitude ``mscale(factor, mscale) / mscale(factor, mscale_all_dim)``;
* per head: ``s = scale * (q_nope . k_nope + q_pe . k_pe)``, causal with bottom-right alignment
  (python/minisgl/attention/fa.py:155: the ``n_new`` new tokens are the last of the history),
  ``o = softmax(s) v``; ``out = W_o [o_1 .. o_H]``.

``absorbed=True`` computes the same attention the decode kernels compute -- scores
``(q_nope W_UK) . c + q_pe . k_pe`` and ``o = (softmax . c) W_UV^T`` -- a different route to the
same numbers (tests pin the two against each other in float64).

``round_bf16=True`` rounds to bfloat16 at the points where the product keeps bf16 tensors
(every projection output, the normed latent, the roped dims, the attention output), so that
the comparison with the GPU path measures the kernels and GEMMs, not where rounding happens.

All dims are read from the weight shapes, so tiny layers work (the brute-force pins use them).
"""

from __future__ import annotations

import math
from typing import Optional

import torch


def yarn_mscale(factor: float, mscale: float) -> float:
    """The YaRN paper's attention factor ``0.1 * mscale * ln(factor) + 1`` (1 when ``factor <= 1``)."""
    return 1.0 if factor <= 1.0 else 0.1 * mscale * math.log(factor) + 1.0


def rope_inv_freq(rotary_dim: int, base: float, rope_scaling: Optional[dict] = None):
    """float64 ``inv_freq [d/2]`` and the cos/sin amplitude (rotary.py:23-24, 92-111)."""
    i = torch.arange(rotary_dim // 2, dtype=torch.float64)
    inv = base ** (-2.0 * i / rotary_dim)
    rs = dict(rope_scaling or {})
    kind = rs.get("rope_type", rs.get("type", "default"))
    if kind == "default":
        return inv, 1.0
    assert kind == "yarn", kind
    factor = float(rs["factor"])
    orig = float(rs["original_max_position_embeddings"])
    # dims that turn fewer than beta_slow times over the original context are interpolated
    # (divided by factor), those turning more than beta_fast times are kept; linear ramp between
    corr = lambda n: rotary_dim * math.log(orig / (n * 2.0 * math.pi)) / (2.0 * math.log(base))  # noqa: E731
    lo = max(math.floor(corr(float(rs.get("beta_fast", 32.0)))), 0)
    hi = min(math.ceil(corr(float(rs.get("beta_slow", 1.0)))), rotary_dim // 2 - 1)
    ramp = torch.clamp((i - lo) / max(hi - lo, 1), 0.0, 1.0)
    inv = inv * (1.0 - ramp) + inv / factor * ramp
    amp = 1.0
    if rs.get("mscale") is not None and rs.get("mscale_all_dim") is not None:
        amp = yarn_mscale(factor, float(rs["mscale"])) / yarn_mscale(factor, float(rs["mscale_all_dim"]))
    return inv, amp


def rope(x: torch.Tensor, positions: torch.Tensor, inv_freq: torch.Tensor, amp: float, interleaved: bool):
    """Rotate ``x [T, ..., d]`` (float64) by ``positions [T] * inv_freq``."""
    ang = positions.to(torch.float64)[:, None] * inv_freq[None, :]  # [T, d/2]
    shape = (x.shape[0],) + (1,) * (x.dim() - 2) + (ang.shape[1],)
    cos, sin = (ang.cos() * amp).reshape(shape), (ang.sin() * amp).reshape(shape)
    out = torch.empty_like(x)
    if interleaved:
        a, b = x[..., 0::2], x[..., 1::2]
        out[..., 0::2] = a * cos - b * sin
        out[..., 1::2] = b * cos + a * sin
    else:
        h = x.shape[-1] // 2
        a, b = x[..., :h], x[..., h:]
        out[..., :h] = a * cos - b * sin
        out[..., h:] = b * cos + a * sin
    return out


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps) * w


def mla_layer(
    x: torch.Tensor,
    positions: torch.Tensor,
    n_new: int,
    weights: dict,
    *,
    num_heads: int,
    rope_dim: int,
    rope_theta: float,
    rope_scaling: Optional[dict] = None,
    interleaved: bool = True,
    eps: float = 1e-6,
    scale: Optional[float] = None,
    round_bf16: bool = False,
    absorbed: bool = False,
    dtype: torch.dtype = torch.float64,
) -> torch.Tensor:
    """Layer output ``[n_new, hidden]`` for the last ``n_new`` tokens of one request.

    ``x [L, hidden]`` holds the request's whole history (prefix first), ``positions [L]`` their
    positions; ``weights`` maps q_a, q_a_norm, q_b, kv_a, kv_a_norm, kv_b, o to
    ``[out, in]`` matrices (and norm vectors). ``scale`` defaults to ``1/sqrt(nope + rope)``.
    """
    W = {k: v.to(dtype) for k, v in weights.items()}
    H = num_heads
    rnd = (lambda t: t.to(torch.bfloat16).to(dtype)) if round_bf16 else (lambda t: t)  # noqa: E731
    x = x.to(dtype)
    L = x.shape[0]
    r = W["kv_a_norm"].shape[0]  # latent width
    qk = W["q_b"].shape[0] // H  # nope + rope
    nope = qk - rope_dim
    dv = W["kv_b"].shape[0] // H - nope
    if scale is None:
        scale = 1.0 / math.sqrt(qk)
    inv_freq, amp = rope_inv_freq(rope_dim, rope_theta, rope_scaling)

    xn = x[L - n_new :]
    pos_new = positions[L - n_new :]
    q = rnd(rnd(rms_norm(rnd(xn @ W["q_a"].T), W["q_a_norm"], eps)) @ W["q_b"].T).view(n_new, H, qk)
    q_nope = q[..., :nope]
    q_pe = rnd(rope(q[..., nope:], pos_new, inv_freq.to(dtype), amp, interleaved))
    kv = rnd(x @ W["kv_a"].T)
    c = rnd(rms_norm(kv[:, :r], W["kv_a_norm"], eps))  # [L, r]
    k_pe = rnd(rope(kv[:, r:], positions, inv_freq.to(dtype), amp, interleaved))  # [L, rope]
    kvb = W["kv_b"].view(H, nope + dv, r)
    w_uk, w_uv = kvb[:, :nope], kvb[:, nope:]  # [H, nope, r], [H, dv, r]

    # causal, bottom-right aligned: new token i (at row L - n_new + i) sees rows 0 .. L - n_new + i
    rows = torch.arange(L)
    mask = rows[None, :] <= (L - n_new + torch.arange(n_new))[:, None]  # [n_new, L]
    s_pe = torch.einsum("thd,ld->htl", q_pe, k_pe)
    if absorbed:
        q_lat = torch.einsum("thn,hnr->htr", q_nope, w_uk)
        s = (torch.einsum("htr,lr->htl", q_lat, c) + s_pe) * scale
    else:
        k_nope = rnd(torch.einsum("lr,hnr->hln", c, w_uk))  # [H, L, nope]
        s = (torch.einsum("thn,hln->htl", q_nope, k_nope) + s_pe) * scale
    s = s.masked_fill(~mask[None], float("-inf"))
    p = torch.softmax(s, dim=-1)  # [H, n_new, L]
    if absorbed:
        o = torch.einsum("htl,lr,hvr->thv", p, c, w_uv)
    else:
        v = rnd(torch.einsum("lr,hvr->hlv", c, w_uv))  # [H, L, dv]
        o = torch.einsum("htl,hlv->thv", p, v)
    o = rnd(o).reshape(n_new, H * dv)
    return rnd(o @ W["o"].T)


def mla_layer_loops(x, positions, n_new, weights, *, num_heads, rope_dim, rope_theta, interleaved=True, eps=1e-6):
    """The same layer as scalar Python loops (float64, no YaRN, no rounding): tiny inputs only."""
    W = {k: v.to(torch.float64).tolist() for k, v in weights.items()}
    H = num_heads
    X = x.to(torch.float64).tolist()
    P = [float(p) for p in positions.tolist()]
    L, hidden = len(X), len(X[0])
    r = len(W["kv_a_norm"])
    qk = len(W["q_b"]) // H
    nope = qk - rope_dim
    dv = len(W["kv_b"]) // H - nope
    scale = 1.0 / math.sqrt(qk)

    def matvec(M, v):
        return [sum(M[i][j] * v[j] for j in range(len(v))) for i in range(len(M))]

    def norm(v, w):
        ms = sum(e * e for e in v) / len(v)
        return [v[i] / math.sqrt(ms + eps) * w[i] for i in range(len(v))]

    def rot(v, pos):
        d = len(v)
        out = list(v)
        for i in range(d // 2):
            th = pos * rope_theta ** (-2.0 * i / d)
            a, b = (2 * i, 2 * i + 1) if interleaved else (i, i + d // 2)
            out[a] = v[a] * math.cos(th) - v[b] * math.sin(th)
            out[b] = v[b] * math.cos(th) + v[a] * math.sin(th)
        return out

    keys, vals = [], []  # per token: per head k [qk], v [dv]
    for t in range(L):
        kv = matvec(W["kv_a"], X[t])
        c = norm(kv[:r], W["kv_a_norm"])
        kpe = rot(kv[r:], P[t])
        kt, vt = [], []
        for h in range(H):
            row0 = h * (nope + dv)
            kt.append([sum(W["kv_b"][row0 + n][j] * c[j] for j in range(r)) for n in range(nope)] + kpe)
            vt.append([sum(W["kv_b"][row0 + nope + n][j] * c[j] for j in range(r)) for n in range(dv)])
        keys.append(kt)
        vals.append(vt)
    outs = []
    for i in range(n_new):
        t = L - n_new + i
        q = matvec(W["q_b"], norm(matvec(W["q_a"], X[t]), W["q_a_norm"]))
        o_all = []
        for h in range(H):
            qh = q[h * qk : h * qk + nope] + rot(q[h * qk + nope : (h + 1) * qk], P[t])
            s = [scale * sum(qh[d] * keys[j][h][d] for d in range(qk)) for j in range(t + 1)]
            m = max(s)
            e = [math.exp(z - m) for z in s]
            tot = sum(e)
            o_all += [sum(e[j] / tot * vals[j][h][n] for j in range(t + 1)) for n in range(dv)]
        outs.append(matvec(W["o"], o_all))
    assert len(outs[0]) == hidden
    return torch.tensor(outs, dtype=torch.float64)
