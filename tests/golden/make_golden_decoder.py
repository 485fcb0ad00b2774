"""Write golden vectors of the verify forward from the reference's ``LanguageModel.extend``.

``oracle/decoder.py`` restates the reference's verify forward (oxr_runtime/language.py:69-104,
201-214, 247-317).  No closed form in the reference's tests pins its bf16 bits, so this script
runs the reference itself on seeded inputs (``decoder_inputs.py``) and stores what it returns:
the final-norm hidden states of the new tokens, the K/V rows the step writes into every layer's
cache, the bf16 logits (language.py:213-214) and their argmax (decode_graph.py:167).

The reference's attention goes to flash-attn (attention.py:96-109), which is absent here; its
own test module, tests/test_language_fused.py, installs a plain PyTorch ``oxr_runtime.attention``
before it imports the language model (test_language_fused.py:17-65).  This script imports that
test module to get the same setup, then uses the ``language`` module it imported.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_golden_decoder.py /root/reference

The committed ``decoder_extend.npz`` is data: checksums of the regenerated inputs, the small
integer inputs, and the reference's outputs.  Nothing from the reference's source is stored.
"""

from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import decoder_inputs as di  # noqa: E402

OUT = HERE / "decoder_extend.npz"


def _reference_language(reference_root: str):
    sys.path.insert(0, reference_root)
    path = Path(reference_root) / "tests" / "test_language_fused.py"
    spec = importlib.util.spec_from_file_location("reference_test_language_fused", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)  # installs the test's attention module, imports oxr_runtime.language
    return module.language, module.LanguageConfig, module.KVCache


def main(reference_root: str) -> None:
    torch.set_num_threads(1)
    language, LanguageConfig, KVCache = _reference_language(reference_root)
    assert language.BLOCK_SIZE == di.BLOCK_SIZE
    out: dict[str, np.ndarray] = {}
    for name, case in di.CASES.items():
        c = di.config(case)
        params = di.parameters(case)
        inputs = di.step_inputs(case)
        k_init, v_init = di.caches(inputs)
        ref_config = LanguageConfig(**vars(c))
        model = language.LanguageModel(ref_config, max_positions=case["max_positions"])
        model.load_state_dict({k: v.float() for k, v in params.items()}, strict=True)
        model.fuse_projections()
        model = model.to(torch.bfloat16).eval().requires_grad_(False)
        model.cast_rope(torch.bfloat16)

        cache = KVCache(ref_config, case["num_blocks"], dtype=torch.bfloat16, device=torch.device("cpu"))
        cache.k.copy_(k_init)
        cache.v.copy_(v_init)
        s = case["tokens_per_seq"]
        ids = torch.from_numpy(inputs["ids"])
        batch = language.ExtendBatch(
            model.embed_tokens(ids), torch.from_numpy(inputs["positions"]), torch.from_numpy(inputs["slots"]),
            torch.from_numpy(inputs["seq_lens"]), torch.from_numpy(inputs["table"]), s,
        )
        with torch.inference_mode():
            hidden = model.extend(batch, cache)
            logits = model.logits(hidden)
        predicted = logits.argmax(dim=-1)
        flat = (c.num_layers, -1, c.num_kv_heads, c.head_dim)
        slots = torch.from_numpy(inputs["slots"])
        rec = {
            "checksum": np.array(di.checksum(params, k_init, v_init)),
            "ids": inputs["ids"], "positions": inputs["positions"], "slots": inputs["slots"],
            "seq_lens": inputs["seq_lens"], "table": inputs["table"],
            "hidden": di.bits(hidden), "logits": di.bits(logits), "predicted": predicted.numpy().astype(np.int64),
            "k_rows": di.bits(cache.k.view(flat)[:, slots]), "v_rows": di.bits(cache.v.view(flat)[:, slots]),
        }
        for key, value in rec.items():
            out[f"{name}/{key}"] = value
        print(f"{name}: hidden {tuple(hidden.shape)}, predicted {predicted.tolist()}")
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
