"""CPU oracle for the S6 latent decode-attention path. TEST INFRASTRUCTURE ONLY.

This package is a numpy restatement of the reference PyTorch semantics of the S6 serving
path (``hla/vllm_latent/s6_ops.py``, ``hla/vllm_latent/s6_layer.py``, ``hla/latent/register.py``).
Every function cites the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker or as the timed CPU baseline. The product path (the package
``hybrid-latent-attention_amd``) never imports it: there is no CPU fallback.

Parity pinning (each function and what pins it):

* ``token_requests``, ``history_lengths``, ``num_kv_splits``, ``S6Workspace`` sizes,
  ``latent_rope_table`` row 0: the reference's own known-answer tables, transcribed into
  ``tests/golden/known_answers.json``.
* ``history_attention``, ``chunk_attention``, ``window_decode`` / ``window_history``,
  ``merge_states`` / ``merge_lse``: brute-force float64 per-token softmax loops on tiny inputs
  and the joint-softmax identity (a merge of two partial softmaxes equals one softmax over
  the union of their keys); the window forms are pinned by the closed form only (the
  reference's tests never call them).
* ``latent_rope``: the closed form ``x*cos + rotate_half(x)*sin`` against an explicit pairwise
  rotation, ``table[0] = [1..1, 0..0]``, and norm preservation of the rotation.
* ``absorb``: a textbook batched GEMM checked against ``numpy.einsum`` in float64.
* slot mapping / block-table expansion: the reference's bit-exact rollout-cache expectation.
"""
