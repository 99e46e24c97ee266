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


def test_layer_op_argument_errors_are_reported():
    """The layer ops' C-ABI checks reject bad shapes and strides before any device work."""
    from minisgl_amd.kernel import lib

    so = lib.load_library()
    buf = ctypes.create_string_buffer(64 * 1024 + 16)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16  # 16-byte aligned host address, never dereferenced
    rc = so.mla_rmsnorm_bf16(p, 512, p, 2, 7, 1e-6, p, 512, None)
    assert rc != 0 and b"multiple of 8" in so.mla_last_error()
    rc = so.mla_rmsnorm_bf16(p, 500, p, 2, 512, 1e-6, p, 512, None)
    assert rc != 0 and b"strides" in so.mla_last_error()
    rc = so.mla_latent_rows_bf16(p, 576, p, p, p, 0, 4, 1e-6, 1, p, 576, None)
    assert rc != 0 and b"max_position" in so.mla_last_error()
    rc = so.mla_latent_rows_bf16(p, 512, p, p, p, 16, 4, 1e-6, 1, p, 576, None)
    assert rc != 0 and b">= 576" in so.mla_last_error()
    rc = so.mla_q_rope_bf16(p, 192, 192, 4, 2, p, p, 16, 1, p, 128, 64, None, 0, 0, None)
    assert rc != 0 and b"heads of 192" in so.mla_last_error()
    rc = so.mla_q_rope_bf16(p, 384, 192, 4, 2, p, p, 16, 1, p, 128, 64, p + 2, 128, 512, None)
    assert rc != 0 and b"nope_out" in so.mla_last_error()
    rc = so.mla_qkv_a_rows_bf16(p, 2112, 1530, p, p, p, p, 16, 4, 1e-6, 1, p, 576, None)
    assert rc != 0 and b"q_rank" in so.mla_last_error()
    assert so.mla_rmsnorm_bf16(None, 0, None, 0, 8, 1e-6, None, 0, None) == 0  # no rows: nothing to do


def test_prefill_entry_argument_errors_are_reported():
    """The prefill entry points' C-ABI checks (layouts the kernel cannot address) fire before any
    device work."""
    from minisgl_amd.kernel import lib

    so = lib.load_library()
    buf = ctypes.create_string_buffer(1 << 20)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 256  # aligned host address, never dereferenced
    H, row = 16, 16 * 256 + 64

    def strided(k_rope_off, k_head=256, k_rope_head=0, row_stride=row, page_size=64):
        return so.mla_prefill_strided_bf16(p, H * 192, 192, p, row_stride, k_head, p + k_rope_off, k_rope_head,
                                          p + 256, row_stride, 256, 4, page_size, p, 4, p, p, 2, 10, H, 0.1, p,
                                          H * 128, 128, None, 0, None)

    # rope dims before a head's nope dims (head 15's rope would sit 256 B before its nope start)
    rc = strided(2 * 256 * (H - 1) - 256)
    assert rc != 0 and b"rope dims" in so.mla_last_error()
    rc = strided(2 * 256 * H, row_stride=15 * 256)  # rows too short for 16 heads
    assert rc != 0 and b"hold 16 heads" in so.mla_last_error()
    rc = strided(2 * 256 * H, page_size=32)
    assert rc != 0 and b"page_size" in so.mla_last_error()
    rc = so.mla_prefill_gather_bf16(p, 576, 4, 48, p, 4, p, p, 2, 3, p, 512, p, 64, 256, p, 3, None)
    assert rc != 0 and b"power of two" in so.mla_last_error()
    rc = so.mla_prefill_gather_bf16(p, 576, 4, 16, p, 4, p, p, 2, 3, p, 512, p, 64, 256, p, 2, None)
    assert rc != 0 and b"seg_pt_stride" in so.mla_last_error()
    rc = so.mla_prefill_gather_bf16(p, 576, 4, 16, p, 4, p, p, 2, 3, p, 500, p, 64, 256, p, 3, None)
    assert rc != 0 and b"strides" in so.mla_last_error()
    assert so.mla_prefill_gather_bf16(None, 0, 0, 1, None, 0, None, None, 0, 0, None, 0, None, 0, 0, None, 0,
                                      None) == 0  # no requests: nothing to do
