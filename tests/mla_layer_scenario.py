"""A serving sequence for the MLA layer tests: chunked prefill, decode steps and a prefill
continuing after decode, driven the way mini-sglang's scheduler drives a layer (a ``Batch`` with
``positions`` / ``out_loc`` from the token table, ``prepare_metadata``, then ``forward`` inside
``ctx.forward_batch``), and the oracle's output for every step."""

from __future__ import annotations

from typing import Dict, List, Sequence, Tuple

import torch

from minisgl_amd.core import Batch, Req
from oracle import ref_mla_layer as RL

# (phase, {request: new tokens}); decode steps extend every listed request by one token
STEPS: List[Tuple[str, Dict[int, int]]] = [
    ("prefill", {0: 40, 1: 25}),
    ("prefill", {0: 30, 2: 17}),  # second chunk of request 0 over its 40-token prefix
    ("decode", {0: 1, 1: 1, 2: 1}),
    ("decode", {0: 1, 1: 1, 2: 1}),
    ("prefill", {1: 20}),  # new input after decoding: attends the decoded tokens' K/V too
    ("decode", {0: 1, 1: 1, 2: 1}),
]


class TorchLayerOps:
    """fp32 torch versions of the layer's elementwise steps (``HipLayerOps``' contract), for
    running the layer's glue on the CPU and as the GPU kernels' fp32 reference."""

    @staticmethod
    def rms_norm(x, w, eps):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()).to(x.dtype)

    @staticmethod
    def rope(x, positions, cos_sin, interleaved):
        d = x.shape[-1]
        cs = cos_sin[positions.long()]
        shape = (x.shape[0],) + (1,) * (x.dim() - 2) + (d // 2,)
        cos, sin = cs[:, : d // 2].reshape(shape), cs[:, d // 2 :].reshape(shape)
        xf = x.float()
        if interleaved:
            x1, x2 = xf[..., 0::2], xf[..., 1::2]
            return torch.stack((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).flatten(-2).to(x.dtype)
        x1, x2 = xf[..., : d // 2], xf[..., d // 2 :]
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)

    @classmethod
    def latent_rows(cls, kv, w, positions, cos_sin, eps, interleaved):
        return torch.cat((cls.rms_norm(kv[:, :512], w, eps), cls.rope(kv[:, 512:], positions, cos_sin, interleaved)),
                         dim=-1)

    @classmethod
    def qkv_a_rows(cls, qkv_a, q_rank, q_w, kv_w, positions, cos_sin, eps, interleaved):
        return (cls.rms_norm(qkv_a[:, :q_rank], q_w, eps),
                cls.latent_rows(qkv_a[:, q_rank:], kv_w, positions, cos_sin, eps, interleaved))

    @classmethod
    def q_rope(cls, q, positions, cos_sin, interleaved, pe_out, nope_out=None):
        pe_out.copy_(cls.rope(q[..., 128:], positions, cos_sin, interleaved))
        if nope_out is not None:
            nope_out.copy_(q[..., :128])


def scaled_steps(factor: int) -> List[Tuple[str, Dict[int, int]]]:
    return [(ph, {r: (e * factor if ph == "prefill" else e) for r, e in st.items()}) for ph, st in STEPS]


def total_lens(steps) -> Dict[int, int]:
    tot: Dict[int, int] = {}
    for ph, st in steps:
        if ph == "free":
            continue
        for r, e in st.items():
            tot[r] = tot.get(r, 0) + e
    return tot


def token_table(lens: Dict[int, int], page_size: int, gen: torch.Generator, spare_pages: int = 2):
    """Token table (one token location per column) over shuffled whole pages, and the page count."""
    need = {r: -(-L // page_size) for r, L in lens.items()}
    num_pages = sum(need.values()) + spare_pages
    width = -(-max(n * page_size for n in need.values()) // 32) * 32
    tt = torch.zeros((max(lens) + 2, width), dtype=torch.int32)
    starts = torch.randperm(num_pages, generator=gen)[: sum(need.values())] * page_size
    off = 0
    for r, n in sorted(need.items()):
        tt[r, : n * page_size] = (starts[off : off + n].unsqueeze(1) + torch.arange(page_size)).flatten().to(torch.int32)
        off += n
    return tt, num_pages


def run(layer, ctx, backend, x_hist: Dict[int, torch.Tensor], steps, tt: torch.Tensor, device, alloc=None):
    """Run ``steps`` through ``layer``; yields (phase, [(request, new tokens)], tokens per request
    after the step, output [T, hidden]). With ``alloc`` (a PagedTokenTable over ``ctx.page_table``)
    pages are allocated step by step as the scheduler does, and a ("free", {r: 0}) step returns a
    finished request's pages."""
    cached = {r: 0 for r in x_hist}
    for phase, st in steps:
        if phase == "free":
            for r in st:
                alloc.free(r, cached[r])
            continue
        order = sorted(st)
        reqs = [Req(table_idx=r, cached_len=cached[r], device_len=cached[r] + st[r]) for r in order]
        batch = Batch(reqs=reqs, phase=phase)
        batch.padded_reqs = reqs
        batch.positions = torch.cat([torch.arange(q.cached_len, q.device_len) for q in reqs]).to(torch.int32).to(device)
        if alloc is not None:
            alloc.allocate_paged(reqs)
            batch.out_loc = alloc.out_loc(reqs)
        else:
            batch.out_loc = torch.cat([tt[q.table_idx, q.cached_len : q.device_len] for q in reqs]).to(device)
        x = torch.cat([x_hist[r][cached[r] : cached[r] + st[r]] for r in order]).to(device)
        backend.prepare_metadata(batch)
        with ctx.forward_batch(batch):
            out = layer.forward(x)
        for r in order:
            cached[r] += st[r]
        yield phase, [(r, st[r]) for r in order], dict(cached), out


def expected(x_hist, new: Sequence[Tuple[int, int]], cached_after: Dict[int, int], weights: dict, **kw):
    """The oracle's output for one step, requests in batch order."""
    outs = []
    for r, e in new:
        L = cached_after[r]
        outs.append(RL.mla_layer(x_hist[r][:L], torch.arange(L), e, weights, **kw))
    return torch.cat(outs)
