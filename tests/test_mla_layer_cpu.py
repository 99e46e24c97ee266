"""The MLA layer's oracle pinned on the CPU, and the product layer's glue checked against it.

Pins of ``oracle/ref_mla_layer.py``:
* brute force: the tensor oracle equals scalar Python loops over a tiny layer (both RoPE layouts);
* the absorbed route (decode's ``q W_UK . c``, ``(p . c) W_UV^T``) equals the decompressed one in
  float64, with YaRN;
* RoPE closed forms: position 0 is the identity, pair norms are kept, scores depend on the
  position difference only, the interleaved layout is the half layout under a permutation;
  YaRN reduces to plain RoPE at factor 1, keeps the fast dims and divides the slow dims by the
  factor, and its attention factor at (32, 1) is ``1 + 0.1 ln 32``;
* RMSNorm on a constant vector.
A planted mistake (the per-head ``W_kvb`` split read K/V-major instead of head-major) must fail
the brute-force pin.

The product layer (``minisgl_amd.layers``) runs on the CPU here in float32 over a dense stand-in
pool and backend (the HIP kernels need a GPU); its chunked-prefill / decode / continued-prefill
outputs must match the float64 oracle.
"""

from __future__ import annotations

import math

import pytest
import torch

from minisgl_amd.config import MLAConfig
from minisgl_amd.core import Context, reset_global_ctx, set_global_ctx
from minisgl_amd.layers import MLAAttentionLayer, MLALayerConfig, MLAWeights, rope_cos_sin_cache, softmax_mscale
from oracle import ref_mla as R
from oracle import ref_mla_layer as RL

import mla_layer_scenario as S

KIMI_YARN = (
    ("rope_type", "yarn"),
    ("factor", 32.0),
    ("original_max_position_embeddings", 4096),
    ("beta_fast", 1.0),
    ("beta_slow", 1.0),
    ("mscale", 1.0),
    ("mscale_all_dim", 1.0),
)
DSV3_YARN = (
    ("rope_type", "yarn"),
    ("factor", 40.0),
    ("original_max_position_embeddings", 4096),
    ("beta_fast", 32.0),
    ("beta_slow", 1.0),
    ("mscale", 1.0),
    ("mscale_all_dim", 1.0),
)


def _tiny_weights(gen, H, hidden, q_lora, r, rope, nope, dv):
    f = lambda *s: torch.randn(s, generator=gen, dtype=torch.float64) / math.sqrt(s[-1])  # noqa: E731
    return {
        "q_a": f(q_lora, hidden),
        "q_a_norm": 1 + 0.1 * torch.randn(q_lora, generator=gen, dtype=torch.float64),
        "q_b": f(H * (nope + rope), q_lora),
        "kv_a": f(r + rope, hidden),
        "kv_a_norm": 1 + 0.1 * torch.randn(r, generator=gen, dtype=torch.float64),
        "kv_b": f(H * (nope + dv), r),
        "o": f(hidden, H * dv),
    }


TINY = dict(H=2, hidden=10, q_lora=7, r=8, rope=4, nope=6, dv=5)


@pytest.mark.parametrize("interleaved", [True, False])
def test_oracle_matches_scalar_loops(interleaved):
    gen = torch.Generator().manual_seed(3)
    W = _tiny_weights(gen, **TINY)
    L, n_new = 6, 4
    x = torch.randn((L, TINY["hidden"]), generator=gen, dtype=torch.float64)
    pos = torch.tensor([0, 1, 2, 5, 9, 13])
    kw = dict(num_heads=TINY["H"], rope_dim=TINY["rope"], rope_theta=100.0, interleaved=interleaved)
    got = RL.mla_layer(x, pos, n_new, W, **kw)
    want = RL.mla_layer_loops(x, pos, n_new, W, **kw)
    torch.testing.assert_close(got, want, atol=1e-12, rtol=1e-12)


def test_planted_kv_b_split_mistake_fails_the_loops():
    gen = torch.Generator().manual_seed(4)
    W = _tiny_weights(gen, **TINY)
    H, nope, dv, r = TINY["H"], TINY["nope"], TINY["dv"], TINY["r"]
    x = torch.randn((5, TINY["hidden"]), generator=gen, dtype=torch.float64)
    pos = torch.arange(5)
    kw = dict(num_heads=H, rope_dim=TINY["rope"], rope_theta=100.0)
    # the mistake: rows of W_kvb taken as [nope + dv, H] instead of [H, nope + dv]
    bad = dict(W, kv_b=W["kv_b"].view(nope + dv, H, r).transpose(0, 1).reshape(H * (nope + dv), r))
    assert not torch.allclose(RL.mla_layer(x, pos, 3, bad, **kw), RL.mla_layer_loops(x, pos, 3, W, **kw), atol=1e-6)


@pytest.mark.parametrize("scaling", [None, DSV3_YARN])
def test_absorbed_equals_decompressed(scaling):
    gen = torch.Generator().manual_seed(5)
    W = _tiny_weights(gen, H=4, hidden=48, q_lora=24, r=32, rope=8, nope=16, dv=12)
    L = 40
    x = torch.randn((L, 48), generator=gen, dtype=torch.float64)
    pos = torch.arange(L) * 97  # long positions exercise the interpolated dims
    kw = dict(num_heads=4, rope_dim=8, rope_theta=10000.0, rope_scaling=dict(scaling or ()))
    for n_new in (1, 7, L):
        a = RL.mla_layer(x, pos, n_new, W, absorbed=True, **kw)
        d = RL.mla_layer(x, pos, n_new, W, absorbed=False, **kw)
        torch.testing.assert_close(a, d, atol=1e-12, rtol=1e-12)


def test_rope_closed_forms():
    gen = torch.Generator().manual_seed(6)
    inv, amp = RL.rope_inv_freq(64, 50000.0)
    assert amp == 1.0
    q = torch.randn((1, 64), generator=gen, dtype=torch.float64)
    k = torch.randn((1, 64), generator=gen, dtype=torch.float64)
    for inter in (True, False):
        torch.testing.assert_close(RL.rope(q, torch.tensor([0]), inv, 1.0, inter), q, atol=0, rtol=0)
        rq = RL.rope(q, torch.tensor([1234]), inv, 1.0, inter)
        pairs = lambda t: (t[0, 0::2] ** 2 + t[0, 1::2] ** 2) if inter else (t[0, :32] ** 2 + t[0, 32:] ** 2)  # noqa: E731
        torch.testing.assert_close(pairs(rq), pairs(q), atol=1e-12, rtol=1e-12)
        for m, n, s in ((5, 2, 100), (4000, 17, 3000)):
            d1 = (RL.rope(q, torch.tensor([m]), inv, 1.0, inter) * RL.rope(k, torch.tensor([n]), inv, 1.0, inter)).sum()
            d2 = (RL.rope(q, torch.tensor([m + s]), inv, 1.0, inter) * RL.rope(k, torch.tensor([n + s]), inv, 1.0, inter)).sum()
            assert abs(float(d1 - d2)) < 1e-9
    # interleaved == halves under the (evens, odds) permutation
    perm = torch.cat((torch.arange(0, 64, 2), torch.arange(1, 64, 2)))
    p = torch.tensor([777])
    torch.testing.assert_close(
        RL.rope(q, p, inv, 1.0, True)[:, perm], RL.rope(q[:, perm], p, inv, 1.0, False), atol=1e-12, rtol=1e-12
    )


def test_yarn_closed_forms():
    base, d = 10000.0, 64
    plain, _ = RL.rope_inv_freq(d, base)
    same, amp1 = RL.rope_inv_freq(d, base, {"rope_type": "yarn", "factor": 1.0, "original_max_position_embeddings": 4096})
    torch.testing.assert_close(same, plain, atol=0, rtol=1e-15)
    assert amp1 == 1.0
    inv, amp = RL.rope_inv_freq(d, base, dict(DSV3_YARN))
    assert amp == 1.0  # mscale == mscale_all_dim
    # beta_fast 32 -> dims below floor(10.47) = 10 keep their frequency; beta_slow 1 -> from ceil(22.5) = 23 on, / 40
    corr = lambda n: d * math.log(4096 / (n * 2 * math.pi)) / (2 * math.log(base))  # noqa: E731
    lo, hi = math.floor(corr(32)), math.ceil(corr(1))
    assert (lo, hi) == (10, 23)
    torch.testing.assert_close(inv[:lo + 1], plain[:lo + 1], atol=0, rtol=0)
    torch.testing.assert_close(inv[hi:], plain[hi:] / 40.0, atol=0, rtol=1e-15)
    assert torch.all((inv[lo + 1 : hi] < plain[lo + 1 : hi]) & (inv[lo + 1 : hi] > plain[lo + 1 : hi] / 40.0))
    assert RL.yarn_mscale(32.0, 1.0) == pytest.approx(1.0 + 0.1 * math.log(32.0), abs=1e-15)
    assert softmax_mscale(KIMI_YARN) == pytest.approx(1.0 + 0.1 * math.log(32.0), abs=1e-15)
    assert softmax_mscale(None) == 1.0


@pytest.mark.parametrize("scaling", [None, KIMI_YARN, DSV3_YARN])
def test_product_cos_sin_cache_matches_oracle(scaling):
    """The layer's fp32 cos/sin table against the oracle's float64 angles (rotary.py:27-31 builds
    the table in fp32 the same way: position x inv_freq, then cos and sin)."""
    cache = rope_cos_sin_cache(64, 8192, 50000.0, scaling).double()
    inv, amp = RL.rope_inv_freq(64, 50000.0, dict(scaling or ()))
    ang = torch.arange(8192, dtype=torch.float64)[:, None] * inv[None, :]
    torch.testing.assert_close(cache[:, :32], ang.cos() * amp, atol=2e-3, rtol=0)
    torch.testing.assert_close(cache[:, 32:], ang.sin() * amp, atol=2e-3, rtol=0)
    torch.testing.assert_close(cache[:100, :32], ang[:100].cos() * amp, atol=1e-5, rtol=0)


@pytest.mark.parametrize("interleaved", [True, False])
def test_torch_layer_ops_match_oracle(interleaved):
    """The fp32 torch ops that stand in for the HIP ones on the CPU (and are the GPU kernels'
    fp32 reference) against the oracle's float64 rope / RMSNorm."""
    gen = torch.Generator().manual_seed(7)
    cache = rope_cos_sin_cache(64, 8192, 50000.0, KIMI_YARN)
    inv, amp = RL.rope_inv_freq(64, 50000.0, dict(KIMI_YARN))
    pos = torch.randint(0, 8192, (33,), generator=gen)
    kv = torch.randn((33, 576), generator=gen)
    w = 1 + 0.1 * torch.randn(512, generator=gen)
    got = S.TorchLayerOps.latent_rows(kv, w, pos, cache, 1e-6, interleaved).double()
    torch.testing.assert_close(got[:, :512], RL.rms_norm(kv[:, :512].double(), w.double(), 1e-6), atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(got[:, 512:], RL.rope(kv[:, 512:].double(), pos, inv, amp, interleaved), atol=5e-3,
                               rtol=0)
    q = torch.randn((33, 5, 192), generator=gen)
    pe, nope = torch.empty((33, 5, 64)), torch.empty((5, 33, 128))
    S.TorchLayerOps.q_rope(q, pos, cache, interleaved, pe, nope.transpose(0, 1))
    torch.testing.assert_close(pe.double(), RL.rope(q[..., 128:].double(), pos, inv, amp, interleaved), atol=5e-3,
                               rtol=0)
    assert torch.equal(nope.transpose(0, 1), q[..., :128])


def test_rms_norm_closed_form():
    x = torch.full((3, 512), 0.25)
    w = torch.linspace(0.5, 1.5, 512)
    want = (w * 0.25 / math.sqrt(0.0625 + 1e-6)).expand(3, 512)
    torch.testing.assert_close(S.TorchLayerOps.rms_norm(x, w, 1e-6), want)
    torch.testing.assert_close(RL.rms_norm(x.double(), w.double(), 1e-6), want.double())


# ---------------------------------------------------------------- product layer on a CPU stand-in


class _DensePool:
    """Dense stand-in for the MLA pool: latent rows indexed by token location."""

    def __init__(self, num_tokens):
        self.latent = torch.zeros((num_tokens, 576))

    def store_kv(self, k, v, out_loc, layer_id):
        assert k.dim() == 2
        self.latent[out_loc.long()] = k.float()


class _DenseBackend:
    """Dense stand-in for the MLA backend's contract: store the latent rows, then decode over them
    (``q [B, H, 576]`` -> ``[B, H, 512]``) or causal prefill over the keys decompressed from them with
    the layer's registered ``W_kvb``."""

    def __init__(self, pool, tt, scale):
        self.pool, self.tt, self.scale = pool, tt, scale
        self.kv_b = {}

    def prepare_metadata(self, batch):
        batch.attn_metadata = None

    def register_kv_b(self, layer_id, kv_b):
        self.kv_b[layer_id] = kv_b

    def forward(self, q, k, v, layer_id, batch):
        self.pool.store_kv(k, v, batch.out_loc, layer_id)
        outs, off = [], 0
        for req in batch.reqs:
            rows = self.tt[req.table_idx, : req.device_len].long()
            e = req.extend_len
            qi = q[off : off + e].float().transpose(0, 1)  # [H, e, D]
            H = qi.shape[0]
            kv = self.pool.latent[rows]
            if batch.is_decode:
                o, _ = R._attend(qi, kv.expand(H, -1, -1), kv[:, :512].expand(H, -1, -1), self.scale)
            else:
                L = req.device_len
                w = self.kv_b[layer_id].float().view(H, 256, 512)
                k_nope = torch.matmul(kv[None, :, :512], w[:, :128].transpose(1, 2))  # [H, L, 128]
                vh = torch.matmul(kv[None, :, :512], w[:, 128:].transpose(1, 2))
                kh = torch.cat((k_nope, kv[None, :, 512:].expand(H, -1, -1)), dim=-1)
                mask = torch.arange(L)[None, :] <= (L - e + torch.arange(e))[:, None]
                o, _ = R._attend(qi, kh, vh, self.scale, mask[None])
            outs.append(o.transpose(0, 1))
            off += e
        return torch.cat(outs).to(q.dtype)


@pytest.mark.parametrize("scaling", [None, KIMI_YARN])
def test_product_layer_on_dense_stand_in(scaling):
    reset_global_ctx()
    gen = torch.Generator().manual_seed(9)
    H = 4
    attn = MLAConfig(num_heads=H, softmax_mscale=softmax_mscale(scaling))
    cfg = MLALayerConfig(attn=attn, hidden_size=64, q_lora_rank=48, rope_theta=50000.0, max_position=4096,
                         rope_scaling=scaling)
    weights = MLAWeights.random(cfg, gen, "cpu", dtype=torch.float32)
    layer = MLAAttentionLayer(0, cfg, weights, ops=S.TorchLayerOps())
    lens = S.total_lens(S.STEPS)
    tt, num_pages = S.token_table(lens, 16, gen)
    ctx = Context(page_size=16)
    set_global_ctx(ctx)
    ctx.page_table = tt
    pool = _DensePool(num_pages * 16)
    backend = _DenseBackend(pool, tt, attn.softmax_scale)
    ctx.kv_cache, ctx.attn_backend = pool, backend
    x_hist = {r: torch.randn((L, 64), generator=gen) for r, L in lens.items()}
    Wd = {k: getattr(weights, k).double() for k in ("q_a", "q_a_norm", "q_b", "kv_a", "kv_a_norm", "kv_b", "o")}
    kw = dict(num_heads=H, rope_dim=64, rope_theta=50000.0, rope_scaling=dict(scaling or ()), interleaved=True,
              scale=attn.softmax_scale)
    try:
        for phase, new, after, out in S.run(layer, ctx, backend, x_hist, S.STEPS, tt, "cpu"):
            want = S.expected(x_hist, new, after, Wd, **kw)
            torch.testing.assert_close(out.double(), want, atol=1e-3, rtol=1e-3, msg=f"{phase} {new}")
    finally:
        reset_global_ctx()
