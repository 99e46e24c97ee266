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
    assert slots <= ctas + B and slots <= 2 * ctas
    return plan, pieces


@pytest.mark.parametrize("ps", [1, 16, 64, 128])
@pytest.mark.parametrize("ctas", [1, 7, 256])
def test_plan_covers_every_token(ps, ctas):
    rng = np.random.default_rng(ps * 1000 + ctas)
    lens = rng.integers(0, 3000, size=13).tolist() + [0, 1, 64, 65]
    # pieces have no length limit; one CTA holds at most MAX_CTA_BLOCKS blocks
    total_blocks = sum(-(-L // lib.PLAN_BLOCK) for L in lens)
    if -(-total_blocks // lib.MAX_CTA_BLOCKS) > ctas:
        with pytest.raises(lib.MLAKernelError):
            lib.decode_plan(lens, ps, ctas)
        return
    _check(lens, ps, ctas)


@pytest.mark.parametrize("ps", [1, 16, 64, 128])
def test_plan_piece_cap(ps):
    """``max_piece_pages`` caps the pages a piece touches; every further piece of a request starts a
    new CTA."""
    lens = [5000, 3000, 64, 1]
    plan, slots = lib.decode_plan(lens, ps, 64, max_piece_pages=128)
    max_blk = (128 * ps if ps <= lib.PLAN_BLOCK else 127 * ps) // lib.PLAN_BLOCK
    for _, b, t0, t1 in plan_pieces(plan, 64, lens):
        assert -(-(t1 - t0) // lib.PLAN_BLOCK) <= max_blk
    with pytest.raises(lib.MLAKernelError, match="cannot hold"):
        lib.decode_plan([100000], ps, 2, max_piece_pages=128)


def test_plan_is_balanced_for_kimi_decode():
    rng = np.random.default_rng(0)
    lens = rng.integers(1024, 8193, size=64).tolist()
    plan, pieces = _check(lens, 64, 256)
    load = np.zeros(256)
    for w, b, t0, t1 in pieces:
        load[w] += -(-(t1 - t0) // 64) + 2
    assert load.max() <= 1.15 * load.mean()


def test_plan_long_context():
    _check([131072, 32768, 70000], 64, 256)
    # pieces of any length at page size 1 too: one CTA takes a whole 5000-token request
    plan, pieces = _check([5000, 3000], 1, 1)
    assert [(t0, t1) for _, _, t0, t1 in pieces] == [(0, 5000), (0, 3000)]


def test_plan_rejects_impossible():
    # 200000 tokens = 3125 blocks > 2 * MAX_CTA_BLOCKS
    with pytest.raises(lib.MLAKernelError, match="cannot hold"):
        lib.decode_plan([200000], 1, 2)
    # more than MAX_CTA_REQUESTS requests in one CTA
    with pytest.raises(lib.MLAKernelError, match="cannot hold"):
        lib.decode_plan([1] * (lib.MAX_CTA_REQUESTS + 1), 64, 1)


def _backend(ps, num_ctas=256):
    import torch

    from minisgl_amd.attention.mla import MLAAttnBackend
    from minisgl_amd.config import MLAConfig
    from minisgl_amd.core import Context, reset_global_ctx, set_global_ctx
    from minisgl_amd.kvcache import create_kvcache_pool

    reset_global_ctx()
    ctx = Context(page_size=ps)
    set_global_ctx(ctx)
    ctx.kv_cache = create_kvcache_pool(MLAConfig(num_layers=1, num_heads=16), 4, ps, torch.bfloat16, "cpu")
    be = MLAAttnBackend(MLAConfig(num_layers=1, num_heads=16), num_ctas=num_ctas)
    reset_global_ctx()
    return be


@pytest.mark.parametrize("ps", [1, 64])
def test_backend_plans_kimi_batch_on_one_round(ps):
    """The Kimi-K2 batch (336807 tokens) fits one CTA per compute unit at any page size."""
    from minisgl_amd.benchmark.layer import decode_lens

    lens = decode_lens()
    be = _backend(ps)
    plan, slots, ctas = be._plan(lens)
    assert ctas == 256 and plan.shape[0] == ctas * lib.PLAN_CTA_INTS + len(lens) * lib.PLAN_REQ_INTS
    assert slots <= 2 * ctas


@pytest.mark.parametrize("ps", [1, 64])
@pytest.mark.parametrize("max_bs", [160, 256])
def test_capture_grid_holds_any_replayable_batch(ps, max_bs):
    """init_capture_graph at the reference's defaults (max_seq_len 131072, graph batch sizes up to
    160 / 256, python/minisgl/engine/graph.py:58-62) sizes the captured plan grid from max_bs *
    max_seq_len, not from the pool: requests that share radix-cache prefix pages can hold more
    tokens in all than the pool has, and every replayable batch must plan on the captured grid.
    Replayed batches are padded with empty ranges; eager batches plan on their own workspace."""
    be = _backend(ps)
    bs_list = [1, 2, 4] + list(range(8, max_bs + 1, 8))
    be.init_capture_graph(max_seq_len=131072, bs_list=bs_list)
    assert be.capture_ctas * lib.MAX_CTA_BLOCKS * lib.PLAN_BLOCK >= max_bs * 131072
    assert be.capture_ctas == {160: 1024, 256: 2048}[max_bs]
    graph_ws = be.ws_graph[0]
    assert graph_ws.shape[0] == 2 * be.capture_ctas
    pool_tokens = be.kvcache.num_pages * ps
    rng = np.random.default_rng(ps)
    # shared-prefix batch: every request 100k-131k tokens long (far more tokens than the pool holds)
    lens = rng.integers(100_000, 131_073, size=max_bs).tolist()
    assert sum(lens) > 2_000_000 > pool_tokens
    plan, slots, grid = be._plan(lens, be.capture_ctas)
    assert grid == be.capture_ctas and slots <= graph_ws.shape[0]
    assert plan.shape[0] == grid * lib.PLAN_CTA_INTS + max_bs * lib.PLAN_REQ_INTS
    pieces = plan_pieces(plan, grid, lens)
    assert sum(t1 - t0 for *_, t0, t1 in pieces) == sum(lens)
    # the Kimi-K2 decode batch replayed: the same grid, the ranges past the planned ones empty
    lens = rng.integers(1024, 8193, size=max_bs).tolist()
    plan, slots, grid = be._plan(lens, be.capture_ctas)
    assert grid == be.capture_ctas
    cta = plan[: grid * 4].reshape(grid, 4)
    used = int((cta[:, 0] < max_bs).sum())
    assert used <= 256 and (cta[used:] == np.array([max_bs, 0, max_bs, 0])).all()
    assert sum(t1 - t0 for *_, t0, t1 in plan_pieces(plan, grid, lens)) == sum(lens)
    # a replayed batch with few tokens
    plan, slots, grid = be._plan([1] * 8, be.capture_ctas)
    cta = plan[: grid * 4].reshape(grid, 4)
    assert (cta[8:] == np.array([8, 0, 8, 0])).all()
    # eager batches plan on their own grid and workspace, never on the graphs' one
    big = rng.integers(1024, 8193, size=256).tolist()
    plan, slots, ctas = be._plan(big)
    ws = be._eager_workspace(slots)
    assert ws[0].shape[0] >= slots and be.ws_graph[0] is graph_ws


def test_capture_plan_padding_is_a_suffix():
    """The kernels stop a CTA's loop over ranges w, w + grid, ... at the first padding range: the
    padding of a plan laid out for a larger grid must be the suffix of the ranges, and no range
    before it may be empty-by-padding."""
    be = _backend(64)
    be.init_capture_graph(max_seq_len=131072, bs_list=[1, 64, 160])
    rng = np.random.default_rng(3)
    for B in (1, 64, 160):
        lens = rng.integers(1, 131_073, size=B).tolist()
        plan, _, grid = be._plan(lens, be.capture_ctas)
        first = plan[: grid * 4].reshape(grid, 4)[:, 0]
        pad = np.nonzero(first >= B)[0]
        assert len(pad) == 0 or (pad == np.arange(pad[0], grid)).all()


def test_backend_device_bytes():
    """backend_device_bytes: what the backend holds beside the pool, known before the pool is sized."""
    from minisgl_amd.attention.mla import backend_device_bytes, decode_workspace_bytes, prefill_scratch_bytes

    H = 64
    b = backend_device_bytes(H, 256, max_running_req=256, max_seq_len=131072, prefill_scratch_rows=65536)
    # 256 x 131072 tokens need 2048 plan ranges: 4096 slots
    assert b == prefill_scratch_bytes(H, 65536) + decode_workspace_bytes(H, 4096)
    assert decode_workspace_bytes(H, 1) == H * (1024 + 4)
    g = backend_device_bytes(H, 256, 256, 131072, 65536, graph_max_bs=160)
    assert g == b + decode_workspace_bytes(H, 2048) + 4 * (1024 * 4 + 160 * 3)


def test_retired_eager_workspace_is_kept_until_its_decode_completes():
    """A grown eager workspace replaces the old one only in the backend's bookkeeping: the old buffers
    stay referenced until the event recorded after the decode that last used them has completed."""
    import torch


    class Fence:
        def __init__(self):
            self.done = False

        def query(self):
            return self.done

    be = _backend(64)
    ws_a = be._eager_workspace(10)
    assert ws_a[0].shape[0] == 2 * be.num_ctas and ws_a[0].dtype == torch.bfloat16
    fence = Fence()
    be.ws_eager_fence = fence  # what forward records after a decode on ws_a
    ws_b = be._eager_workspace(10 * be.num_ctas)  # growth
    assert ws_b[0] is not ws_a[0] and ws_b[0].shape[0] == 10 * be.num_ctas
    assert len(be.ws_retired) == 1 and be.ws_retired[0][0][0] is ws_a[0], "the old workspace is fenced"
    be._eager_workspace(5)
    assert len(be.ws_retired) == 1, "still in use: kept"
    fence.done = True
    be._eager_workspace(5)
    assert be.ws_retired == [], "its decode completed: released"
    # a workspace that no decode used (no fence) is released at once
    be._eager_workspace(20 * be.num_ctas)
    assert be.ws_retired == []


def test_prefill_passes_hold_whole_requests_within_the_scratch():
    """Passes are runs of consecutive whole requests whose 64-row pages fit the scratch; a request
    longer than the scratch is a pass of its own; seg_first counts pages from the pass start."""
    from minisgl_amd.attention.mla import prefill_passes

    lens = [128, 400, 1300, 200, 41, 127, 1]
    passes = prefill_passes(lens, 512)
    assert passes == [(0, 1, [0]), (1, 2, [0]), (2, 3, [0]), (3, 7, [0, 4, 5, 7])]
    covered = [r for r0, r1, _ in passes for r in range(r0, r1)]
    assert covered == list(range(len(lens)))
    for r0, r1, first in passes:
        pages = [-(-L // 64) for L in lens[r0:r1]]
        assert first == [sum(pages[:i]) for i in range(len(pages))]
        assert r1 - r0 == 1 or sum(pages) * 64 <= 512
    assert prefill_passes(lens, 1 << 20) == [(0, 7, [0, 2, 9, 30, 34, 35, 37])]
    assert prefill_passes([], 512) == []
