"""Write the small seeded golden fixtures under tests/golden/ (run on the CPU).

Inputs are drawn with the same seeds as the benchmarks (0: lengths and page
tables, 1: queries, 2: KV); expected outputs come from the float64 oracle
(oracle/ref_mla.py). bf16 tensors are stored as their raw uint16 bits.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mini-sglang_amd")]

from minisgl_amd.benchmark.inputs import make_decode_case, page_table_for  # noqa: E402
from oracle import ref_mla as R  # noqa: E402


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def decode_fixture(path: str) -> None:
    case = make_decode_case(3, 16, 16, lens=[1, 37, 150], extra_pages=2, seed=0)
    o, lse = R.mla_decode(case.q, case.kv_pool, case.page_table, case.lens, R.DEFAULT_SCALE, dtype=torch.float64)
    np.savez_compressed(
        path,
        q_bits=bits(case.q),
        kv_bits=bits(case.kv_pool),
        page_table=case.page_table.numpy(),
        seq_lens=np.asarray(case.lens, dtype=np.int32),
        page_size=np.int32(case.page_size),
        scale=np.float64(R.DEFAULT_SCALE),
        o=o.float().numpy(),
        lse=lse.numpy(),
    )


def page_table_fixture(path: str) -> None:
    gen = torch.Generator().manual_seed(0)
    ps, rows, width, num_pages = 16, 6, 256, 64
    lens = [1, 17, 48, 200, 255, 100]
    tt = torch.zeros((rows, width), dtype=torch.int32)
    starts = (torch.randperm(num_pages, generator=gen) * ps).to(torch.int32)
    off = 0
    for r, L in enumerate(lens):
        n = -(-L // ps)
        toks = (starts[off : off + n].unsqueeze(1) + torch.arange(ps, dtype=torch.int32)).flatten()
        tt[r, : n * ps] = toks
        off += n
    table_idx = torch.tensor([3, 5, 0, 1], dtype=torch.int32)
    max_len = max(lens[i] for i in table_idx.tolist())
    pt = R.page_table_from_tokens(tt, table_idx, max_len, ps)
    np.savez_compressed(path, token_table=tt.numpy(), table_idx=table_idx.numpy(), max_seqlen_k=np.int32(max_len),
                        page_size=np.int32(ps), page_table=pt.numpy())


def main() -> None:
    torch.set_num_threads(min(8, torch.get_num_threads()))
    decode_fixture(os.path.join(HERE, "decode_small.npz"))
    page_table_fixture(os.path.join(HERE, "page_table_small.npz"))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
