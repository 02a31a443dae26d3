"""Speculative-decoding verification on the HIP kernels (reference: src/miniserve/spec)."""
