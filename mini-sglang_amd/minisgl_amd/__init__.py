"""MI355X-native MLA attention backend with mini-sglang's backend interface.

Subpackages mirror the reference's layout for the hot path only:
``attention`` (BaseAttnBackend + the MLA backend), ``kvcache`` (the MLA KV
pool), ``kernel`` (libmla_amd.so via ctypes), ``core`` (Req/Batch/Context).
"""
