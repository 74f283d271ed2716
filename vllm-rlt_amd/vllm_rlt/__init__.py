"""MI355X (gfx950) ``hip`` backend for vllm-rlt's depth-aware paged KV path.

This package mirrors the reference's module names (``vllm_rlt.attention``,
``vllm_rlt.kernels``, ``vllm_rlt.worker.metadata``, ``vllm_rlt.core``) for the
hot path only, so the callers' imports and call signatures stay unchanged.
Importing it touches no GPU.
"""

__version__ = "0.1.0"
