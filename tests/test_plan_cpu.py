"""Host split-KV planner (libmla_amd's mla_decode_plan) invariants, on the CPU."""

from __future__ import annotations

import numpy as np
import pytest

from minisgl_amd.attention.mla import plan_pieces
from minisgl_amd.kernel import lib


def _check(lens, ps, ctas):
    plan, slots = lib.decode_plan(lens, ps, ctas)
    B = len(lens)
    req = plan[ctas * 4 :].reshape(B, 3) if B else np.zeros((0, 3), np.int32)
    pieces = plan_pieces(plan, ctas, lens)
    # every token of every request is covered exactly once, in order
    for b, L in enumerate(lens):
        mine = [(t0, t1, w) for (w, bb, t0, t1) in pieces if bb == b]
        covered = 0
        for t0, t1, _ in mine:
            assert t0 == covered and t1 > t0
            covered = t1
        assert covered == L
        assert req[b, 1] == len(mine)
        if mine:
            ws = [w for *_, w in mine]
            assert ws == list(range(req[b, 0], req[b, 0] + len(mine))), "pieces of a request sit in consecutive CTAs"
            assert all(t0 % lib.PLAN_BLOCK == 0 for t0, _, _ in mine)
    # split requests own disjoint, dense slot ranges
    used = []
    for b in range(B):
        if req[b, 1] >= 2:
            used += list(range(req[b, 2], req[b, 2] + req[b, 1]))
    assert sorted(used) == list(range(slots))
    assert slots <= ctas + B
    return plan, pieces


@pytest.mark.parametrize("ps", [1, 16, 64, 128])
@pytest.mark.parametrize("ctas", [1, 7, 256])
def test_plan_covers_every_token(ps, ctas):
    rng = np.random.default_rng(ps * 1000 + ctas)
    lens = rng.integers(0, 3000, size=13).tolist() + [0, 1, 64, 65]
    # a piece may touch at most MAX_PIECE_PAGES pages, and every further piece of a
    # request starts a new CTA, so the batch needs 1 + sum(pieces_b - 1) CTAs at least
    max_blk = (lib.MAX_PIECE_PAGES * ps if ps <= lib.PLAN_BLOCK else (lib.MAX_PIECE_PAGES - 1) * ps) // lib.PLAN_BLOCK
    max_blk = min(max_blk, lib.MAX_CTA_BLOCKS)
    needed = 1 + sum(max(0, -(-(-(-L // lib.PLAN_BLOCK)) // max_blk) - 1) for L in lens)
    # and one CTA holds at most MAX_CTA_BLOCKS blocks
    total_blocks = sum(-(-L // lib.PLAN_BLOCK) for L in lens)
    if needed > ctas or -(-total_blocks // lib.MAX_CTA_BLOCKS) > ctas:
        with pytest.raises(lib.MLAKernelError):
            lib.decode_plan(lens, ps, ctas)
        return
    _check(lens, ps, ctas)


def test_plan_is_balanced_for_kimi_decode():
    rng = np.random.default_rng(0)
    lens = rng.integers(1024, 8193, size=64).tolist()
    plan, pieces = _check(lens, 64, 256)
    load = np.zeros(256)
    for w, b, t0, t1 in pieces:
        load[w] += -(-(t1 - t0) // 64) + 2
    assert load.max() <= 1.15 * load.mean()


def test_plan_long_context_and_piece_cap():
    lens = [131072, 32768, 70000]
    _check(lens, 64, 256)
    # page size 1: a piece may touch at most 1024 pages (tokens)
    plan, pieces = _check([5000, 3000], 1, 64)
    assert max(t1 - t0 for _, _, t0, t1 in pieces) <= 1024


def test_plan_rejects_impossible():
    with pytest.raises(lib.MLAKernelError):
        lib.decode_plan([100000], 1, 2)


def test_backend_plans_more_ctas_for_small_pages():
    """With pages under 32 tokens a piece holds at most MAX_PIECE_PAGES tokens, so the Kimi-K2 batch
    (336807 tokens) needs more pieces than 256 CTAs: the backend doubles the CTA count (the extra
    CTAs run as further rounds) instead of failing; page size 64 keeps one CTA per compute unit."""
    import torch

    from minisgl_amd.attention.mla import MLAAttnBackend
    from minisgl_amd.benchmark.layer import decode_lens
    from minisgl_amd.config import MLAConfig
    from minisgl_amd.core import Context, reset_global_ctx, set_global_ctx
    from minisgl_amd.kvcache import create_kvcache_pool

    lens = decode_lens()
    with pytest.raises(lib.MLAKernelError, match="cannot hold"):
        lib.decode_plan(lens, 1, 256)
    for ps, want in ((1, 512), (64, 256)):
        reset_global_ctx()
        ctx = Context(page_size=ps)
        set_global_ctx(ctx)
        ctx.kv_cache = create_kvcache_pool(MLAConfig(num_layers=1), 4, ps, torch.bfloat16, "cpu")
        be = MLAAttnBackend(MLAConfig(num_layers=1), num_ctas=256)
        plan, slots, ctas = be._plan(lens, 256)
        assert ctas == want and plan.shape[0] == ctas * lib.PLAN_CTA_INTS + len(lens) * lib.PLAN_REQ_INTS
        reset_global_ctx()
