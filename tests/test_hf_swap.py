"""swap_to_nmsparse on real Hugging Face decoders (transformers' LlamaForCausalLM
and Qwen3ForCausalLM, tiny random-init configs, no download), called as the
reference's Qwen3 benchmark calls it on the inner decoder
(benchmarks/bench_qwen_31_14b_fp16_fixed_ptx.py:518-532).

CPU: count, module paths, attributes and buffer digests equal what the
reference's own swap produced on the same models (tests/golden/swap_hf_models.json,
written by tests/golden/make_hf_swap_golden.py), and the models' own forward
(prefill: the kept dense weights) is unchanged. GPU: the unmodified model code
decodes through the swapped modules (one-row inputs: the sparse GEMV, q/k/v and
gate/up tied into one launch each) and matches the same model with the sparse
weights scattered to dense, in fp32.
"""
import hashlib
import json

import pytest
import torch

from conftest import GOLDEN, say
from spmv_decode_amd import NmSparseLinear, swap_to_nmsparse

transformers = pytest.importorskip("transformers")

FIX = json.loads((GOLDEN / "swap_hf_models.json").read_text())


def hf_model(arch, **over):
    """The fixture's model of `arch`, random init from torch.manual_seed(0)."""
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM

    cfg = {**FIX["meta"]["config"], **over}
    torch.manual_seed(0)
    if arch == "llama":
        return LlamaForCausalLM(LlamaConfig(**cfg)).eval()
    return Qwen3ForCausalLM(Qwen3Config(**cfg)).eval()


def _sha(t):
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


@pytest.mark.parametrize("name", sorted(FIX["models"]))
def test_swap_of_a_transformers_model_matches_the_reference(name):
    case = FIX["models"][name]
    model = hf_model(case["arch"])
    ids = torch.randint(0, FIX["meta"]["config"]["vocab_size"], (1, 7), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        before = model(input_ids=ids).logits
    decoder = getattr(model, "model", model)  # as the reference benchmark does
    count = swap_to_nmsparse(decoder, case["M"], "cpu")
    assert count == case["count"]
    got = [(p, m) for p, m in model.named_modules() if isinstance(m, NmSparseLinear)]
    assert [p for p, _ in got] == [e["path"] for e in case["linears"]]
    for (path, mod), e in zip(got, case["linears"]):
        assert (mod.h, mod.w, mod.block_width, mod.vec_width) == (e["h"], e["w"], e["block_width"], e["vec_width"])
        assert _sha(mod.mat_data.view(torch.int16)) == e["mat_data_sha256"], path
        assert _sha(mod.mat_index) == e["mat_index_sha256"], path
        assert (mod.weight is not None) == e["has_dense_weight"], path
    with torch.no_grad():  # a multi-token forward runs the kept dense weights, as in the reference
        after = model(input_ids=ids).logits
    assert torch.equal(after, before)
    at = decoder.layers[0].self_attn
    assert at.q_proj.__dict__["_siblings"].members == [at.q_proj, at.k_proj, at.v_proj]


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(FIX["models"]))
def test_transformers_model_decodes_through_the_swap(gpu, name, monkeypatch):
    """Prefill (8 tokens: the small-batch SpMM, no dense weight kept) and 6
    greedy decode steps through the model's own forward and cache; each step's
    q/k/v and gate/up run as one grouped launch per layer; logits within fp16
    tolerance of the masked dense twin in fp32."""
    from spmv_decode_amd import hip_spmv

    case = FIX["models"][name]
    model = hf_model(case["arch"], num_hidden_layers=4).to("cuda", torch.float16)
    decoder = model.model
    n = swap_to_nmsparse(decoder, case["M"], "cuda", seed=3, init="device", keep_dense=False)
    assert n == 7 * 4
    twin = hf_model(case["arch"], num_hidden_layers=4).to("cuda", torch.float32)
    twin.load_state_dict({k: v.float() for k, v in model.state_dict().items() if ".mat_" not in k}, strict=False)
    with torch.no_grad():
        for blk_s, blk_t in zip(decoder.layers, twin.model.layers):
            for sub in ("self_attn", "mlp"):
                for pname, mod in getattr(blk_s, sub).named_children():
                    if isinstance(mod, NmSparseLinear):
                        getattr(getattr(blk_t, sub), pname).weight.copy_(mod.to_dense(torch.float32))
    launches = []
    real = hip_spmv.nmsparse_gemv_grouped
    monkeypatch.setattr(hip_spmv, "nmsparse_gemv_grouped", lambda *a, **k: launches.append(1) or real(*a, **k))
    ids = torch.randint(0, 512, (1, 8), generator=torch.Generator().manual_seed(2)).cuda()
    say(f"{name}: transformers decode through the swapped modules")
    with torch.no_grad():
        out_s = model(input_ids=ids, use_cache=True)
        out_t = twin(input_ids=ids, use_cache=True)
        assert not launches  # the prompt is not one row: no grouped decode launch
        for step in range(6):
            ls, lt = out_s.logits[:, -1].float(), out_t.logits[:, -1]
            rel = float((ls - lt).norm() / lt.norm())
            assert torch.isfinite(ls).all() and rel < 1e-2, (step, rel)
            nxt = torch.argmax(lt, dim=-1, keepdim=True)  # teacher-forced by the fp32 twin's choice
            out_s = model(input_ids=nxt, past_key_values=out_s.past_key_values, use_cache=True)
            out_t = twin(input_ids=nxt, past_key_values=out_t.past_key_values, use_cache=True)
            assert len(launches) == 2 * 4 * (step + 1)  # q/k/v and gate/up: one launch each per layer
