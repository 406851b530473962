"""KV structures and transfer backends (mirrors the reference's layover/kv/)."""
