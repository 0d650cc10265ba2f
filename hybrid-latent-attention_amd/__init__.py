"""MI355X (gfx950) implementation of the S6 latent decode-attention path of hybrid-latent-attention.

``s6_ops`` and ``s6_layer`` keep the operator and layer interfaces of ``hla/vllm_latent/s6_ops.py`` and
``hla/vllm_latent/s6_layer.py``; every op runs hand-written HIP kernels from ``libhla_s6.so`` through the C ABI of
``include/hla_s6.h``. The directory name is not a Python identifier: import it with
``importlib.import_module('hybrid-latent-attention_amd')`` with the repository root on ``sys.path``.
``rollout_cache`` gathers a finished request's committed rows and writes its ``s6-rollout-cache-v1`` snapshot (the
reference's own loader reads it back); ``history_gemm`` is
the differentiable history attention over contiguous rows (multi-query for K-hop replay, single-query for the HF
engine); ``batched_engine`` is the HF rolling engine's joint attention over history rows and the current chunk.
"""
from . import _lib, batched_engine, history_gemm, rollout_cache, s6_layer, s6_ops

__all__ = ['_lib', 'batched_engine', 'history_gemm', 'rollout_cache', 's6_layer', 's6_ops']
