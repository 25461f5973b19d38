"""Compressed checkpoints and real pruned weights (f3): the shared mask of an
N:M-pruned dense weight is recovered exactly, the packed buffers reproduce the
weight bit for bit, and they round-trip through state_dict / torch.save."""
import io

import numpy as np
import pytest
import torch

from oracle import nm_oracle as O
from spmv_decode_amd import NmSparseLinear, swap_to_nmsparse
from spmv_decode_amd.decode.model import Decoder, init_weights_, tiny_config
from spmv_decode_amd.nmsparse_linear import index_from_pruned, pack_dense


def _pruned(N, K, M, seed, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    nnz = M // 2
    mi = torch.stack([torch.randperm(M, generator=g)[:nnz].sort().values for _ in range(K // M)]).to(torch.uint8)
    W = (torch.randn(N, K, generator=g) * 0.02).to(dtype)
    mask = torch.from_numpy(O.mask_from_index(mi, nnz, M, K))
    return torch.where(mask, W, torch.zeros((), dtype=dtype)), mi  # pruned entries are +0


@pytest.mark.parametrize("M", [4, 8, 64, 256])
def test_mask_recovered_and_packing_reproduces_the_weight(M):
    W, mi = _pruned(256, 4 * M, M, seed=M)
    got = index_from_pruned(W, M)
    assert got.dtype == torch.uint8 and torch.equal(got, mi)
    md = pack_dense(W, got, M)
    back = O.scatter(md, got, M // 2, M, W.shape[1])
    assert torch.equal(back.view(torch.int16), W.view(torch.int16))  # bit for bit, signed zeros included


@pytest.mark.parametrize("M", [4, 64])
def test_to_dense_is_the_oracle_scatter(M):
    """NmSparseLinear.to_dense equals the oracle's scatter (microbench_triton_torchmv.py:145-164)
    bit for bit, and packing it again gives the module's buffers back."""
    lin = NmSparseLinear(384, 4 * M, M, 3, "cpu")
    dense = lin.to_dense()
    ref = O.scatter(lin.mat_data, lin.mat_index, M // 2, M, 4 * M)
    assert dense.shape == (384, 4 * M) and torch.equal(dense.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(pack_dense(dense, lin.mat_index, M).view(torch.int16), lin.mat_data.view(torch.int16))
    assert lin.to_dense(torch.float32).dtype == torch.float32
    assert torch.equal(lin.to_dense(torch.float32), ref.float())


def test_all_zero_kept_positions_are_completed_deterministically():
    W, mi = _pruned(128, 64, 8, seed=3)
    pos = (torch.arange(mi.numel()) // 4) * 8 + mi.reshape(-1).long()
    W[:, pos[5]] = 0  # a kept column that is zero in every row
    got = index_from_pruned(W, 8)
    assert (got[:, 1:] > got[:, :-1]).all() and got.shape == mi.shape
    back = O.scatter(pack_dense(W, got, 8), got, 4, 8, 64)
    assert torch.equal(back, W)
    assert torch.equal(index_from_pruned(W, 8), got)  # deterministic


def test_not_shared_mask_nm_is_rejected():
    W, _ = _pruned(128, 64, 8, seed=4)
    W[:, :8] = 1.0  # a group with 8 non-zero positions
    with pytest.raises(ValueError, match="not 4:8 sparse"):
        index_from_pruned(W, 8)
    with pytest.raises(ValueError, match="K % M"):
        index_from_pruned(W[:, :60], 8)


def test_state_dict_round_trip_through_torch_save():
    lin = NmSparseLinear(256, 512, 16, seed=7, device="cpu")
    buf = io.BytesIO()
    torch.save(lin.state_dict(), buf)
    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    assert set(sd) >= {"mat_data", "mat_index"}
    new = NmSparseLinear.empty(256, 512, 16, "cpu")
    new.load_state_dict({k: sd[k] for k in ("mat_data", "mat_index")})
    assert torch.equal(new.mat_data.view(torch.int16), lin.mat_data.view(torch.int16))
    assert torch.equal(new.mat_index, lin.mat_index)
    assert (new.h, new.w, new.block_width, new.vec_width) == (lin.h, lin.w, lin.block_width, lin.vec_width)


def test_decoder_checkpoint_round_trip_and_swap_from_pruned_weights():
    cfg = tiny_config()
    torch.manual_seed(0)
    dense = Decoder(cfg)
    init_weights_(dense, seed=2)
    masks = {}
    with torch.no_grad():  # prune every projection to 4:8 with its own shared mask
        for bi, blk in enumerate(dense.layers):
            for sub, names in ((blk.self_attn, ("q_proj", "k_proj", "v_proj", "o_proj")),
                               (blk.mlp, ("gate_proj", "up_proj", "down_proj"))):
                for j, name in enumerate(names):
                    lin = getattr(sub, name)
                    W, mi = _pruned(*lin.weight.shape, 8, seed=100 * bi + j, dtype=torch.float32)
                    lin.weight.copy_(W)
                    masks[(bi, name)] = (W.clone(), mi)
    n = swap_to_nmsparse(dense, 8, "cpu", from_weights=True, keep_dense=False)
    assert n == 7 * cfg.n_layers
    for bi, blk in enumerate(dense.layers):
        for sub, names in ((blk.self_attn, ("q_proj", "k_proj", "v_proj", "o_proj")),
                           (blk.mlp, ("gate_proj", "up_proj", "down_proj"))):
            for name in names:
                mod = getattr(sub, name)
                W, mi = masks[(bi, name)]
                assert torch.equal(mod.mat_index, mi)
                back = O.scatter(mod.mat_data.float(), mod.mat_index, 4, 8, W.shape[1])
                assert torch.equal(back, W.to(torch.float16).float())
    # the swapped model's state_dict restores into a fresh skeleton
    buf = io.BytesIO()
    torch.save(dense.state_dict(), buf)
    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    fresh = Decoder(cfg)
    swap_to_nmsparse(fresh, 8, "cpu", seed=99, keep_dense=False, init="device")
    fresh.load_state_dict(sd)
    for (ka, a), (kb, b) in zip(sorted(dense.state_dict().items()), sorted(fresh.state_dict().items())):
        assert ka == kb and torch.equal(a, b), ka
