"""L1 (single-kernel) decode-step candidates."""
