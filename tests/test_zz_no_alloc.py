"""mla_decode_bf16_noalloc (split-KV partials in the library's fixed device scratch, no workspace
argument) against mla_decode_bf16 with a caller workspace: the same kernels on the same plan, so
outputs and LSEs must agree bit for bit. Two calls in a row, the second on a smaller batch, so the
second reads the scratch the first left behind; plus the size limit, rejected on the host."""

from __future__ import annotations

import pytest
import torch

from minisgl_amd.benchmark.inputs import make_decode_case
from minisgl_amd.kernel import lib
from oracle import ref_mla as R

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _both(case, num_ctas):
    B, H, _ = case.q.shape
    plan_np, slots = lib.decode_plan(case.lens, case.page_size, num_ctas)
    plan = torch.from_numpy(plan_np).to(DEV)
    q, kv, pt, sl = (t.to(DEV) for t in (case.q, case.kv_pool, case.page_table, case.seq_lens))
    ws_o, ws_lse = lib.decode_workspace(slots, H, DEV)
    out_a = torch.full((B, H, 512), float("nan"), dtype=torch.bfloat16, device=DEV)
    lse_a = torch.full((B, H), float("nan"), dtype=torch.float32, device=DEV)
    lib.mla_decode(q, kv, pt, sl, plan, num_ctas, ws_o, ws_lse, R.DEFAULT_SCALE, out_a, lse_a)
    out_b = torch.full((B, H, 512), float("nan"), dtype=torch.bfloat16, device=DEV)
    lse_b = torch.full((B, H), float("nan"), dtype=torch.float32, device=DEV)
    lib.mla_decode_noalloc(q, kv, pt, sl, plan, num_ctas, slots, R.DEFAULT_SCALE, out_b, lse_b)
    torch.cuda.synchronize()
    return slots, out_a.cpu(), lse_a.cpu(), out_b.cpu(), lse_b.cpu()


def test_noalloc_matches_workspace_entry_point():
    first = make_decode_case(16, 64, 64, len_range=(1024, 8192), seed=3)
    second = make_decode_case(5, 16, 16, lens=[1, 100, 3000, 70, 640], seed=4)
    for name, case, ctas in (("first", first, 256), ("second, smaller", second, 7)):
        print(f"[noalloc] {name}: B={len(case.lens)} H={case.q.shape[1]} ps={case.page_size}", flush=True)
        slots, oa, la, ob, lb = _both(case, ctas)
        assert slots > 0, "the case must split requests, so the partials pass through the scratch"
        assert torch.equal(oa.view(torch.int16), ob.view(torch.int16))
        assert torch.equal(la.view(torch.int32), lb.view(torch.int32))
        o_ref, lse_ref = R.mla_decode(case.q, case.kv_pool, case.page_table, case.lens)
        torch.testing.assert_close(ob.float(), o_ref, atol=2e-2, rtol=2e-2)
        torch.testing.assert_close(lb, lse_ref, atol=1e-3, rtol=0.0)


def test_noalloc_rejects_plans_beyond_the_scratch():
    case = make_decode_case(2, 64, 64, lens=[100, 200], seed=5)
    plan = torch.zeros(256 * 4 + 2 * 3, dtype=torch.int32, device=DEV)
    out = torch.empty((2, 64, 512), dtype=torch.bfloat16, device=DEV)
    slots = lib.NOALLOC_MAX_SLOT_HEADS // 64 + 1
    with pytest.raises(lib.MLAKernelError, match="exceed the fixed scratch"):
        lib.mla_decode_noalloc(case.q.to(DEV), case.kv_pool.to(DEV), case.page_table.to(DEV),
                               case.seq_lens.to(DEV), plan, 256, slots, R.DEFAULT_SCALE, out)
