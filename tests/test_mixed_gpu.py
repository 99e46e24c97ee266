"""A ragged batch sharing radix-prefix pages: decode requests and prefill
chunks whose page-table rows reference the same prefix pages, each half
through its HIP kernel (C ABI) against the CPU oracle.

Tolerances: bf16 output atol = rtol = 2e-2; fp32 natural-log LSE atol 1e-3.
"""

from __future__ import annotations

import pytest
import torch

from minisgl_amd.benchmark.inputs import make_mixed_case
from oracle import ref_mla as R

from test_decode_gpu import run_decode
from test_prefill_gpu import run_prefill

pytestmark = pytest.mark.gpu
DEV = "cuda"
O_TOL = dict(atol=2e-2, rtol=2e-2)
LSE_TOL = dict(atol=1e-3, rtol=0.0)


@pytest.mark.parametrize("groups,ps", [(2, 64), (3, 128)])
def test_mixed_shared_prefix(groups, ps):
    m = make_mixed_case(7, 3, 16, ps, (100, 1500), 200, 2 * ps, groups, seed=groups)
    d, p = m.decode, m.prefill
    # rows of one group start with the same page ids
    assert torch.equal(d.page_table[0, :2], d.page_table[groups, :2])
    o_ref, lse_ref = R.mla_decode(d.q, d.kv_pool, d.page_table, d.lens)
    out, lse, _ = run_decode(d.q.to(DEV), d.kv_pool.to(DEV), d.page_table.to(DEV), d.seq_lens.to(DEV), d.lens, ps, 64)
    torch.testing.assert_close(out, o_ref, **O_TOL)
    torch.testing.assert_close(lse, lse_ref, **LSE_TOL)
    o_ref, lse_ref = R.mla_prefill(p.q, p.k_pool, p.v_pool, p.page_table, p.cu_seqlens_q, p.seq_lens_k)
    out, lse = run_prefill(p)
    torch.testing.assert_close(out, o_ref, **O_TOL)
    torch.testing.assert_close(lse, lse_ref, **LSE_TOL)
