"""detllm_amd: MI355X (gfx950) implementation of detllm's per-token decoder
forward pass and logits -> integer-CDF step, bit-identical to the reference
CPU arithmetic.  The compute lives in libdetllm_amd.so (HIP kernels behind
the C ABI of include/detllm.h); these modules mirror the reference's
det-model / det-coder APIs on top of it.
"""

__all__ = ["build", "gguf", "synth"]
