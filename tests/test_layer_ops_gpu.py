"""The MLA layer's elementwise HIP kernels (RMSNorm, latent rows, query RoPE) against their fp32
torch reference and the float64 oracle. Tolerance: atol = rtol = 1e-2 (bf16 outputs: one bf16
ulp is 2^-8 relative); the head-major nope copy is bit-exact."""

from __future__ import annotations

import pytest
import torch

from minisgl_amd.kernel import lib
from minisgl_amd.layers import rope_cos_sin_cache
from oracle import ref_mla_layer as RL

import mla_layer_scenario as S

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = dict(atol=1e-2, rtol=1e-2)
YARN = (("rope_type", "yarn"), ("factor", 32.0), ("original_max_position_embeddings", 4096), ("beta_fast", 1.0),
        ("beta_slow", 1.0), ("mscale", 1.0), ("mscale_all_dim", 1.0))
MAX_POS = 16384


def _bf16(shape, gen, scale=1.0):
    return (torch.randn(shape, generator=gen) * scale).to(torch.bfloat16).to(DEV)


@pytest.mark.parametrize("rows,n,pad", [(0, 512, 0), (1, 512, 0), (37, 1536, 64), (4096, 1536, 0), (5, 7168, 8)])
def test_rmsnorm(rows, n, pad):
    print(f"[rmsnorm] rows={rows} n={n} pad={pad}", flush=True)
    gen = torch.Generator().manual_seed(rows + n)
    x = _bf16((rows, n + pad), gen, 3.0)[:, :n]  # row stride n + pad
    w = _bf16((n,), gen, 0.2) + 1
    out = lib.rmsnorm(x, w, 1e-6)
    torch.cuda.synchronize()
    want = S.TorchLayerOps.rms_norm(x, w, 1e-6)
    torch.testing.assert_close(out.float(), want.float(), **TOL)
    if rows:
        torch.testing.assert_close(out.double().cpu(), RL.rms_norm(x.double().cpu(), w.double().cpu(), 1e-6), **TOL)
    y = x.clone()
    lib.rmsnorm(y, w, 1e-6, out=y)  # in place
    torch.cuda.synchronize()
    assert torch.equal(y, out)


@pytest.mark.parametrize("interleaved", [True, False])
@pytest.mark.parametrize("rows", [1, 64, 3000])
def test_latent_rows(rows, interleaved):
    print(f"[latent_rows] rows={rows} interleaved={interleaved}", flush=True)
    gen = torch.Generator().manual_seed(rows)
    cache = rope_cos_sin_cache(64, MAX_POS, 50000.0, YARN).to(DEV)
    kv = _bf16((rows, 640), gen)[:, :576]
    w = _bf16((512,), gen, 0.1) + 1
    pos = torch.randint(0, MAX_POS, (rows,), generator=gen, dtype=torch.int32)
    pos[0] = MAX_POS - 1
    pos = pos.to(DEV)
    out = lib.latent_rows(kv, w, pos, cache, 1e-6, interleaved)
    torch.cuda.synchronize()
    want = S.TorchLayerOps.latent_rows(kv, w, pos, cache, 1e-6, interleaved)
    torch.testing.assert_close(out.float(), want.float(), **TOL)
    inv, amp = RL.rope_inv_freq(64, 50000.0, dict(YARN))
    k64 = kv.double().cpu()
    torch.testing.assert_close(out[:, :512].double().cpu(), RL.rms_norm(k64[:, :512], w.double().cpu(), 1e-6), **TOL)
    torch.testing.assert_close(out[:, 512:].double().cpu(), RL.rope(k64[:, 512:], pos.cpu(), inv, amp, interleaved),
                               **TOL)


@pytest.mark.parametrize("interleaved", [True, False])
def test_q_rope_decode_layout(interleaved):
    """Decode: rope dims into the absorbed query's last 64 dims, nope dims head-major."""
    T, H = 64, 64
    gen = torch.Generator().manual_seed(11)
    cache = rope_cos_sin_cache(64, MAX_POS, 50000.0, YARN).to(DEV)
    q = _bf16((T, H, 192), gen)
    pos = torch.randint(0, MAX_POS, (T,), generator=gen, dtype=torch.int32).to(DEV)
    q_abs = torch.zeros((T, H, 576), dtype=torch.bfloat16, device=DEV)
    nope_h = torch.zeros((H, T, 128), dtype=torch.bfloat16, device=DEV)
    lib.q_rope(q, pos, cache, interleaved, q_abs[..., 512:], nope_h.transpose(0, 1))
    torch.cuda.synchronize()
    assert torch.equal(nope_h.transpose(0, 1), q[..., :128])
    assert torch.count_nonzero(q_abs[..., :512]) == 0  # untouched
    want = S.TorchLayerOps.rope(q[..., 128:], pos, cache, interleaved)
    torch.testing.assert_close(q_abs[..., 512:].float(), want.float(), **TOL)
    inv, amp = RL.rope_inv_freq(64, 50000.0, dict(YARN))
    torch.testing.assert_close(q_abs[..., 512:].double().cpu(),
                               RL.rope(q[..., 128:].double().cpu(), pos.cpu(), inv, amp, interleaved), **TOL)


def test_q_rope_in_place_prefill_layout():
    T, H = 1000, 16
    gen = torch.Generator().manual_seed(12)
    cache = rope_cos_sin_cache(64, MAX_POS, 50000.0, YARN).to(DEV)
    q = _bf16((T, H, 192), gen)
    ref = q.clone()
    pos = torch.arange(5000, 5000 + T, dtype=torch.int32, device=DEV)
    lib.q_rope(q, pos, cache, True, q[..., 128:])
    torch.cuda.synchronize()
    assert torch.equal(q[..., :128], ref[..., :128])
    torch.testing.assert_close(q[..., 128:].float(), S.TorchLayerOps.rope(ref[..., 128:], pos, cache, True).float(),
                               **TOL)


@pytest.mark.parametrize("heads,interleaved", [(8, False), (20, True), (20, False), (128, True)])
def test_q_rope_head_counts(heads, interleaved):
    """Head counts that do not fill the kernel's 8-head groups (a tensor-parallel shard), both pair
    layouts, in place: the nope dims and the padding past the last head stay untouched."""
    T = 37
    gen = torch.Generator().manual_seed(heads)
    cache = rope_cos_sin_cache(64, MAX_POS, 50000.0, YARN).to(DEV)
    wide = _bf16((T, heads + 1, 192), gen)
    ref = wide.clone()
    q = wide[:, :heads]
    pos = torch.randint(0, MAX_POS, (T,), generator=gen, dtype=torch.int32).to(DEV)
    lib.q_rope(q, pos, cache, interleaved, q[..., 128:])
    torch.cuda.synchronize()
    assert torch.equal(wide[:, heads], ref[:, heads]) and torch.equal(wide[..., :128], ref[..., :128])
    inv, amp = RL.rope_inv_freq(64, 50000.0, dict(YARN))
    torch.testing.assert_close(q[..., 128:].double().cpu(),
                               RL.rope(ref[:, :heads, 128:].double().cpu(), pos.cpu(), inv, amp, interleaved), **TOL)


def test_qkv_a_rows_equals_the_separate_ops():
    """The fused q_a / kv_a rows kernel gives the separate RMSNorm and latent-row kernels' output
    bit for bit (same arithmetic in the same order)."""
    gen = torch.Generator().manual_seed(13)
    cache = rope_cos_sin_cache(64, MAX_POS, 50000.0, YARN).to(DEV)
    for rows, q_rank in ((1, 1536), (64, 1536), (700, 384)):
        qkv = _bf16((rows, q_rank + 576), gen)
        q_w, kv_w = _bf16((q_rank,), gen, 0.1) + 1, _bf16((512,), gen, 0.1) + 1
        pos = torch.randint(0, MAX_POS, (rows,), generator=gen, dtype=torch.int32).to(DEV)
        ref_q = lib.rmsnorm(qkv[:, :q_rank], q_w, 1e-6)
        ref_lat = lib.latent_rows(qkv[:, q_rank:], kv_w, pos, cache, 1e-6, True)
        fused = qkv.clone()
        lat = lib.qkv_a_rows(fused, q_rank, q_w, kv_w, pos, cache, 1e-6, True)
        torch.cuda.synchronize()
        assert torch.equal(fused[:, :q_rank], ref_q) and torch.equal(fused[:, q_rank:], qkv[:, q_rank:])
        assert torch.equal(lat, ref_lat)
