"""HIP kernels of the KV data path (mirrors the reference's layover/kernels/)."""
