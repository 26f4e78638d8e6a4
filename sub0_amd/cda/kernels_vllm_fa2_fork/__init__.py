"""The FA2-fork comparator namespace (reference ``cda/kernels_vllm_fa2_fork``):
``build.load()`` registers ``torch.ops._cda_vllm_fa2_fork_C``."""
