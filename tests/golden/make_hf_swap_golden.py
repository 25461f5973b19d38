"""Write the fixture of swap_to_nmsparse on real Hugging Face decoder models.

Run in the development container only (it needs the reference checkout at
/root/reference, which does not exist on the GPU box, and `transformers`):

    python tests/golden/make_hf_swap_golden.py

It builds tiny random-init `LlamaForCausalLM` and `Qwen3ForCausalLM` models from
configs (no download), imports the reference's own `src/spmv/nmsparse_linear.py`
with NM_KERNEL=triton_ptx (as tests/golden/make_golden.py does), and swaps the
inner decoder exactly as the reference's Qwen3 benchmark does
(benchmarks/bench_qwen_31_14b_fp16_fixed_ptx.py:518-532:
`swap_to_nmsparse(getattr(model, "model", model), m, device)`, default seed),
on the CPU. Recorded, as data only: the swap count and, per swapped Linear, its
module path, attributes and buffer digests. The torch and transformers
versions that produced them are stored alongside.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
from pathlib import Path

import torch

REF = Path(os.environ.get("NM_REFERENCE_ROOT", "/root/reference"))
OUT = Path(__file__).resolve().parent

# name -> (architecture, M); every model: CONFIG (stored in the fixture, which the test builds from)
MODELS = {"llama_L2_d256_M8": ("llama", 8), "qwen3_L2_d256_M16": ("qwen3", 16)}
CONFIG = dict(vocab_size=512, hidden_size=256, intermediate_size=384, num_hidden_layers=2, num_attention_heads=4,
              num_key_value_heads=2, head_dim=64, max_position_embeddings=64)


def hf_model(arch: str):
    """The tiny model of `arch`, random init from torch.manual_seed(0)."""
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM

    torch.manual_seed(0)
    if arch == "llama":
        return LlamaForCausalLM(LlamaConfig(**CONFIG)).eval()
    return Qwen3ForCausalLM(Qwen3Config(**CONFIG)).eval()


def _sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def main():
    import transformers

    os.environ["NM_KERNEL"] = "triton_ptx"
    os.environ["NM_DECODE_ONLY"] = "0"
    os.environ["NM_WEIGHT_CPU"] = "0"
    for p in (REF, REF / "src" / "spmv"):
        if str(p) not in sys.path:
            sys.path.insert(0, str(p))
    import nmsparse_linear as ref  # noqa: E402  (the reference module)

    models = {}
    for name, (arch, M) in MODELS.items():
        model = hf_model(arch)
        decoder = getattr(model, "model", model)
        count = ref.swap_to_nmsparse(decoder, M, "cpu")
        linears = []
        for path, mod in model.named_modules():
            if isinstance(mod, ref.NmSparseLinear):
                linears.append({"path": path, "h": int(mod.h), "w": int(mod.w), "block_width": int(mod.block_width),
                                "vec_width": int(mod.vec_width), "mat_data_sha256": _sha(mod.mat_data.view(torch.int16)),
                                "mat_index_sha256": _sha(mod.mat_index), "has_dense_weight": mod.weight is not None})
        models[name] = {"arch": arch, "M": M, "count": int(count), "linears": linears}
    meta = {"torch": torch.__version__, "transformers": transformers.__version__, "config": CONFIG,
            "source": "src/spmv/nmsparse_linear.py", "call": "benchmarks/bench_qwen_31_14b_fp16_fixed_ptx.py:518-532"}
    (OUT / "swap_hf_models.json").write_text(json.dumps({"meta": meta, "models": models}, indent=1) + "\n")
    print("wrote", OUT / "swap_hf_models.json")


if __name__ == "__main__":
    main()
