"""KV metadata contracts consumed by the hip kernels."""
