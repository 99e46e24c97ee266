"""Measured MI355X peaks beside the published ones: a read-only HBM stream over a buffer larger
than the 256 MB Infinity Cache and a bf16 MFMA loop (kernels in csrc/peaks/mla_peaks.hip, built
into libmla_peaks.so). Times are HIP events on the launch stream."""

from __future__ import annotations

import ctypes
import functools
import os

PEAKS_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmla_peaks.so")
HBM_SPEC_TBPS = 8.0
MFMA_BF16_SPEC_TFLOPS = 2500.0
READ_VARIANTS = {0: "vector loads, 4 in flight", 1: "vector loads, 8 in flight", 2: "vector loads, 16 in flight",
                 3: "vector loads, 8 in flight, non-temporal", 4: "global->LDS DMA, 4-stage ring",
                5: "global->LDS DMA, 4-stage ring, non-temporal"}


@functools.lru_cache(maxsize=None)
def _lib():
    if not os.path.exists(PEAKS_PATH):
        raise RuntimeError(f"{PEAKS_PATH} is missing: build it with `python mini-sglang_amd/build.py`")
    lib = ctypes.CDLL(PEAKS_PATH)
    lib.mla_peaks_hbm_read.restype = ctypes.c_int
    lib.mla_peaks_hbm_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                       ctypes.c_void_p, ctypes.c_void_p]
    lib.mla_peaks_mfma_bf16.restype = ctypes.c_int
    lib.mla_peaks_mfma_bf16.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def _time_ms(fn, stream, reps: int) -> float:
    import torch

    fn()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn()
        b.record(stream)
        b.synchronize()
        best = min(best, a.elapsed_time(b))
    return best


def hbm_read(cu_count: int, gib: int = 4, reps: int = 3) -> dict:
    """Best read bandwidth over the variants and grids (CTAs of 256 threads) of the stream kernel."""
    import torch

    nbytes = gib << 30
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    buf.view(torch.int32).fill_(0x5A5A5A5A)
    stream = torch.cuda.current_stream()
    results = []
    for variant in READ_VARIANTS:
        for mult in ((1,) if variant >= 4 else (1, 2, 4, 8)):
            ctas = cu_count * mult
            sink = torch.empty(ctas * 256, dtype=torch.int32, device="cuda")

            def run():
                rc = _lib().mla_peaks_hbm_read(buf.data_ptr(), nbytes, ctas, variant, sink.data_ptr(),
                                               stream.cuda_stream)
                assert rc == 0, f"mla_peaks_hbm_read failed ({rc})"

            ms = _time_ms(run, stream, reps)
            results.append((nbytes / (ms * 1e-3) / 1e12, variant, ctas))
    del buf
    torch.cuda.empty_cache()
    best = max(results)
    return {
        "tb_per_s": round(best[0], 3),
        "frac_of_spec": round(best[0] / HBM_SPEC_TBPS, 4),
        "spec_tb_per_s": HBM_SPEC_TBPS,
        "best": f"{READ_VARIANTS[best[1]]}, {best[2]} CTAs",
        "bytes": nbytes,
        "by_variant_tb_per_s": {READ_VARIANTS[v]: round(max(r[0] for r in results if r[1] == v), 3)
                                for v in READ_VARIANTS},
    }


def mfma_bf16(cu_count: int, iters: int = 20000, reps: int = 3) -> dict:
    """bf16 dense MFMA throughput: 8 independent 32x32x16 chains per wave, 1 or 2 waves per SIMD."""
    import torch

    stream = torch.cuda.current_stream()
    results = []
    for mult in (1, 2):
        ctas = cu_count * mult
        sink = torch.empty(ctas * 256, dtype=torch.float32, device="cuda")

        def run():
            rc = _lib().mla_peaks_mfma_bf16(iters, ctas, sink.data_ptr(), stream.cuda_stream)
            assert rc == 0, f"mla_peaks_mfma_bf16 failed ({rc})"

        ms = _time_ms(run, stream, reps)
        flops = ctas * 4 * iters * 8 * 32 * 32 * 16 * 2
        results.append((flops / (ms * 1e-3) / 1e12, mult))
    best = max(results)
    return {
        "tflops": round(best[0], 1),
        "frac_of_spec": round(best[0] / MFMA_BF16_SPEC_TFLOPS, 4),
        "spec_tflops": MFMA_BF16_SPEC_TFLOPS,
        "best": f"{best[1]} wave(s) per SIMD, 8 chains of v_mfma_f32_32x32x16_bf16",
    }
