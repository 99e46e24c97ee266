"""Backend registry and prefill/decode dispatch (python/minisgl/attention/__init__.py:19-68,
attention/base.py:37-63) on the CPU, with stand-in backends: the HIP backend itself needs a GPU."""

from __future__ import annotations

from argparse import ArgumentTypeError

import pytest

from minisgl_amd.attention import (
    SUPPORTED_ATTENTION_BACKENDS,
    HybridBackend,
    create_attention_backend,
    supported_backends,
    validate_attn_backend,
)
from minisgl_amd.config import MLAConfig
from minisgl_amd.core import Batch, Req


class _Recorder:
    def __init__(self, name, log):
        self.name, self.log = name, log

    def forward(self, q, k, v, layer_id, batch):
        self.log.append((self.name, "forward"))
        return self.name

    def prepare_metadata(self, batch):
        self.log.append((self.name, "metadata"))

    def init_capture_graph(self, max_seq_len, bs_list):
        self.log.append((self.name, "init_capture"))

    def prepare_for_capture(self, batch):
        self.log.append((self.name, "capture"))

    def prepare_for_replay(self, batch):
        self.log.append((self.name, "replay"))


def test_registry_names():
    assert "mla" in SUPPORTED_ATTENTION_BACKENDS and supported_backends() == ["mla"]
    assert validate_attn_backend("mla") == "mla"
    assert validate_attn_backend("mla,mla") == "mla,mla"
    assert validate_attn_backend("auto") == "auto"
    with pytest.raises(ArgumentTypeError):
        validate_attn_backend("fa")
    with pytest.raises(AssertionError):
        validate_attn_backend("auto", allow_auto=False)
    with pytest.raises(AssertionError):
        create_attention_backend("mla,mla,mla", MLAConfig())


def test_hybrid_dispatch():
    log = []
    hb = HybridBackend(_Recorder("p", log), _Recorder("d", log))
    req = Req(table_idx=0, cached_len=0, device_len=4)
    pre, dec = Batch(reqs=[req], phase="prefill"), Batch(reqs=[req], phase="decode")
    hb.prepare_metadata(pre)
    assert hb.forward(None, None, None, 0, pre) == "p"
    hb.prepare_metadata(dec)
    assert hb.forward(None, None, None, 0, dec) == "d"
    hb.init_capture_graph(4096, [1, 2, 4])
    hb.prepare_for_capture(dec)
    hb.prepare_for_replay(dec)
    assert log == [("p", "metadata"), ("p", "forward"), ("d", "metadata"), ("d", "forward"),
                   ("d", "init_capture"), ("d", "capture"), ("d", "replay")]
