"""MI355X-native (gfx950) speculative-decoding verify step for oxr-inference.

A drop-in for the verify path of NickWilde18/oxr-inference: the modules keep the
reference's call signatures and run hand-written HIP kernels through the C ABI in
``include/oxr_verify.h`` (``liboxr_verify.so``, built by ``build.py``).

- ``speculative``   NgramProposer / accept and their batched device forms
- ``kernels``       qk_norm_rope_store (fused q/k RMSNorm + RoPE + paged KV write)
- ``attention``     paged_extend (multi-query causal paged attention, MFMA)
- ``lm_head``       LM-head GEMM with fused argmax, acceptance and rollback
- ``language``      the Qwen-style decoder's verify forward (``extend``)
- ``kv_cache``      paged KV cache with a runtime block size, page-table packing
- ``decode_graph``  hipGraph capture/replay of the whole verify step

The directory name is not a Python identifier; import it with
``importlib.import_module("oxr-inference_amd")``.
"""

from __future__ import annotations

__all__ = ["speculative", "kernels"]
