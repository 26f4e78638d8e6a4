"""Class-path home of the vLLM backend classes
(drop-in for ``cda/vllm_integration/__init__.py``)."""

__all__: list[str] = []
