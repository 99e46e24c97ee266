"""Synthetic workloads and timing helpers for the MLA kernels."""
