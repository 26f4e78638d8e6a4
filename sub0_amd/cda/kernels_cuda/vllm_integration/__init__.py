"""vLLM attention-backend glue for the MI355X CDA kernels
(drop-in for ``cda/kernels_cuda/vllm_integration/__init__.py``)."""

__all__: list[str] = []
