"""Native kernels of the MLA backend (libmla_amd.so via ctypes)."""

from .lib import (
    MLAKernelError,
    decode_plan,
    device_cu_count,
    load_library,
    mla_decode,
    mla_decode_merge,
    mla_prefill,
    page_table_from_tokens,
    store_rows,
)

__all__ = [
    "MLAKernelError",
    "decode_plan",
    "device_cu_count",
    "load_library",
    "mla_decode",
    "mla_decode_merge",
    "mla_prefill",
    "page_table_from_tokens",
    "store_rows",
]
