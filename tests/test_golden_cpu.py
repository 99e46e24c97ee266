"""CPU checks: the oracle reproduces the committed fixtures, and the C-ABI
library loads and exports every entry point include/mla_amd.h declares."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import torch

from oracle import ref_mla as R

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)


def test_oracle_matches_decode_fixture():
    f = np.load(os.path.join(HERE, "golden", "decode_small.npz"))
    q, kv = _bf16(f["q_bits"]), _bf16(f["kv_bits"])
    o, lse = R.mla_decode(q, kv, torch.from_numpy(f["page_table"]), f["seq_lens"].tolist(), float(f["scale"]))
    assert torch.allclose(o, torch.from_numpy(f["o"]), atol=1e-5, rtol=1e-5)
    assert torch.allclose(lse.double(), torch.from_numpy(f["lse"]), atol=1e-5)


def test_oracle_matches_page_table_fixture():
    f = np.load(os.path.join(HERE, "golden", "page_table_small.npz"))
    got = R.page_table_from_tokens(
        torch.from_numpy(f["token_table"]), torch.from_numpy(f["table_idx"]), int(f["max_seqlen_k"]), int(f["page_size"])
    )
    assert np.array_equal(got.numpy(), f["page_table"])


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "mla_amd.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(mla_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from minisgl_amd.kernel import lib

    names = _declared_symbols()
    assert len(names) >= 8, names
    so = lib.load_library()
    for n in names:
        assert hasattr(so, n), f"{n} missing from {lib.LIB_PATH}"
    assert set(names) == set(lib.SIGNATURES), "ctypes signatures out of sync with the header"
    assert so.mla_abi_version() == lib.ABI_VERSION


def test_host_errors_are_reported():
    from minisgl_amd.kernel import lib

    so = lib.load_library()
    rc = so.mla_decode_plan(None, 1, 64, 4, 1024, None, None, None)
    assert rc != 0 and b"null" in so.mla_last_error()
    lens = (ctypes.c_int32 * 1)(5)
    buf = (ctypes.c_int32 * 16)()
    rc = so.mla_decode_plan(lens, 1, 48, 4, 1024, buf, buf, ctypes.byref(ctypes.c_int32()))
    assert rc == 1 and b"power of two" in so.mla_last_error()
