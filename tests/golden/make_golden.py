"""Write the golden fixtures for synthetic packing and model surgery.

Run in the development container only (it needs the reference checkout at
/root/reference, which does not exist on the GPU box):

    python tests/golden/make_golden.py

It imports the reference's own `src/spmv/nmsparse_linear.py` with
NM_KERNEL=triton_ptx (the shared-mask layout the benchmarks force,
benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:19) and records, as data only:

* `_make_sparse(K, N, M, seed, "cpu")` (src/spmv/nmsparse_linear.py:14-33):
  full mat_data (fp16 bit patterns) and mat_index for small cases, and
  SHA-256 digests of both buffers for Llama-3.1-8B-sized cases.
* `swap_to_nmsparse(model, M, "cpu", seed)` (src/spmv/nmsparse_linear.py:83-144)
  on tiny CPU models in the gpt-fast layout (attention.wqkv/wo,
  feed_forward.w1/w3/w2) and the Hugging Face layout (self_attn.q/k/v/o_proj,
  mlp.gate/up/down_proj): per swapped Linear its path, attributes and buffer
  digests, which fixes the seed order.

Nothing from the reference is copied into the fixtures except these outputs.
The torch version that produced them is stored alongside.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn as nn

REF = Path(os.environ.get("NM_REFERENCE_ROOT", "/root/reference"))
OUT = Path(__file__).resolve().parent

SMALL_CASES = [
    # (K, N_out, M, seed)
    (16, 128, 4, 0),
    (64, 128, 4, 7),
    (64, 128, 8, 0),
    (64, 256, 16, 3),
    (128, 128, 32, 11),
    (256, 128, 64, 5),
    (256, 128, 128, 2),
    (512, 128, 256, 9),
]
DIGEST_CASES = [
    (1024, 3072, 4, 0),      # config 1 shape (Qwen3-0.6B up-proj)
    (4096, 1024, 64, 1),     # Llama k/v proj at 32:64
    (4096, 4096, 64, 0),     # Llama q/o proj at 32:64
    (14336, 4096, 64, 6),    # Llama down proj at 32:64
    (4096, 14336, 4, 4),     # Llama gate/up proj at 2:4
]


def _sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def _import_reference():
    os.environ["NM_KERNEL"] = "triton_ptx"
    os.environ["NM_DECODE_ONLY"] = "0"
    os.environ["NM_WEIGHT_CPU"] = "0"
    for p in (REF, REF / "src" / "spmv"):
        if str(p) not in sys.path:
            sys.path.insert(0, str(p))
    import nmsparse_linear  # noqa: E402  (the reference module)

    return nmsparse_linear


class _GptFastBlock(nn.Module):
    def __init__(self, dim, n_kv, inter):
        super().__init__()
        self.attention = nn.Module()
        self.attention.wqkv = nn.Linear(dim, dim + 2 * n_kv, bias=False)
        self.attention.wo = nn.Linear(dim, dim, bias=False)
        self.feed_forward = nn.Module()
        self.feed_forward.w1 = nn.Linear(dim, inter, bias=False)
        self.feed_forward.w3 = nn.Linear(dim, inter, bias=False)
        self.feed_forward.w2 = nn.Linear(inter, dim, bias=False)


class _HfBlock(nn.Module):
    def __init__(self, dim, n_kv, inter):
        super().__init__()
        self.self_attn = nn.Module()
        self.self_attn.q_proj = nn.Linear(dim, dim, bias=False)
        self.self_attn.k_proj = nn.Linear(dim, n_kv, bias=False)
        self.self_attn.v_proj = nn.Linear(dim, n_kv, bias=False)
        self.self_attn.o_proj = nn.Linear(dim, dim, bias=False)
        self.mlp = nn.Module()
        self.mlp.gate_proj = nn.Linear(dim, inter, bias=False)
        self.mlp.up_proj = nn.Linear(dim, inter, bias=False)
        self.mlp.down_proj = nn.Linear(inter, dim, bias=False)


class _Stack(nn.Module):
    def __init__(self, block_cls, n_layers, dim, n_kv, inter):
        super().__init__()
        self.layers = nn.ModuleList(block_cls(dim, n_kv, inter) for _ in range(n_layers))


def _swap_record(ref_mod, model, M, seed):
    count = ref_mod.swap_to_nmsparse(model, M, "cpu", seed=seed)
    entries = []
    for name, mod in model.named_modules():
        if isinstance(mod, ref_mod.NmSparseLinear):
            entries.append(
                {
                    "path": name,
                    "h": int(mod.h),
                    "w": int(mod.w),
                    "block_width": int(mod.block_width),
                    "vec_width": int(mod.vec_width),
                    "mat_data_shape": list(mod.mat_data.shape),
                    "mat_index_shape": list(mod.mat_index.shape),
                    "mat_data_sha256": _sha(mod.mat_data.view(torch.int16)),
                    "mat_index_sha256": _sha(mod.mat_index),
                    "has_dense_weight": mod.weight is not None,
                }
            )
    return {"count": int(count), "linears": entries}


def main():
    ref_mod = _import_reference()
    meta = {"torch": torch.__version__, "numpy": np.__version__, "source": "src/spmv/nmsparse_linear.py"}

    arrays = {}
    small = []
    for K, N, M, seed in SMALL_CASES:
        md, mi, w, nnz = ref_mod._make_sparse(K, N, M, seed, "cpu")
        tag = f"K{K}_N{N}_M{M}_s{seed}"
        arrays[f"{tag}_mat_data_bits"] = md.view(torch.int16).numpy().view(np.uint16)
        arrays[f"{tag}_mat_index"] = mi.numpy()
        small.append({"K": K, "N": N, "M": M, "seed": seed, "w": int(w), "nnz": int(nnz), "tag": tag})
    np.savez_compressed(OUT / "make_sparse_small.npz", **arrays)

    digests = []
    for K, N, M, seed in DIGEST_CASES:
        md, mi, w, nnz = ref_mod._make_sparse(K, N, M, seed, "cpu")
        digests.append(
            {
                "K": K, "N": N, "M": M, "seed": seed, "w": int(w), "nnz": int(nnz),
                "mat_data_sha256": _sha(md.view(torch.int16)),
                "mat_index_sha256": _sha(mi),
                "mat_index_first_rows": mi[:4].tolist(),
                "mat_data_first": md.view(torch.int16)[0, :8].numpy().view(np.uint16).tolist(),
            }
        )

    swaps = {}
    torch.manual_seed(0)
    gpt = _Stack(_GptFastBlock, 2, 256, 128, 384)
    swaps["gptfast_L2_d256_kv128_i384_M8_seed5"] = _swap_record(ref_mod, gpt, 8, 5)
    torch.manual_seed(0)
    hf = _Stack(_HfBlock, 2, 256, 128, 384)
    swaps["hf_L2_d256_kv128_i384_M4_seed0"] = _swap_record(ref_mod, hf, 4, 0)

    (OUT / "make_sparse.json").write_text(
        json.dumps({"meta": meta, "small": small, "digests": digests}, indent=1) + "\n"
    )
    (OUT / "swap_to_nmsparse.json").write_text(json.dumps({"meta": meta, "models": swaps}, indent=1) + "\n")
    print("wrote", sorted(p.name for p in OUT.iterdir() if p.suffix in (".json", ".npz")))


if __name__ == "__main__":
    main()
