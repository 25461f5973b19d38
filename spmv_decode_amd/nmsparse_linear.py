"""Sparse Linear module and model surgery for the N:M shared-mask GEMV.

Mirrors the reference module API (src/spmv/nmsparse_linear.py):

* `_make_sparse(K, N, M, seed, device)` — synthetic 50% N:M weights, bit-exact
  with the reference (src/spmv/nmsparse_linear.py:14-33, shared-mask branch).
* `NmSparseLinear(N, K, M, seed, device, dense_weight=None)` — buffers
  `mat_data` [w, N] fp16 and `mat_index` [K/M, M/2] uint8, attributes
  `h, w, block_width, vec_width`; decode rows (x.shape[-2] == 1) go through
  `torch.ops.nmsparse.gemv`, longer inputs through dense `F.linear`
  (src/spmv/nmsparse_linear.py:36-68).
* `swap_to_nmsparse(model, M, device, seed=0, block_devices=None)` — replaces
  every attention / MLP Linear of a gpt-fast or Hugging Face decoder stack,
  Linear j getting seed `seed + j` (src/spmv/nmsparse_linear.py:83-144).

Environment, read at import like the reference (src/spmv/nmsparse_linear.py:7-8):
NM_DECODE_ONLY=1 drops dense weights, NM_WEIGHT_CPU=1 keeps them on the host.
Inputs of more than one row (batch > 1): with a dense weight they go through
dense F.linear as in the reference; without one the reference raises
"prefill requires dense weight", and so does a [B, 1, K] input (the op
rejects rows != 1), where this build computes them with the small-batch SpMM
(`torch.ops.nmsparse.spmm`). NM_SPARSE_BATCH=0 restores the reference's
errors; NM_SPARSE_BATCH=1 also sends inputs of up to 128 rows to the SpMM when
a dense weight is present (the matrix-core SpMM's row limit; at the
Llama-3.1-8B shapes it is faster there than hipBLASLt on the dense weight).
NM_SYNTH_INIT=device (this build only) draws the synthetic weights with a
seeded on-device generator instead of the CPU stream — same distribution and
shapes, much faster for 8B+ models, NOT bit-exact with the reference; the
default is the bit-exact CPU stream.

Beyond the reference: `NmSparseLinear.from_dense` / `pack_dense` build the
packed buffers from a real dense weight and a shared N:M mask (a pure gather);
`index_from_pruned` / `NmSparseLinear.from_pruned` recover the shared mask of
an already N:M-pruned dense weight; `NmSparseLinear.to_dense` scatters the
packed weights back (the masked dense weight the module computes with); and
`swap_to_nmsparse(..., from_weights=True)` swaps a pruned checkpoint's own
weights instead of synthetic ones. `NmSparseLinear.empty` builds a module with uninitialised
buffers for `load_state_dict` (the packed buffers are ordinary state_dict
entries, `mat_data` and `mat_index`).
"""
from __future__ import annotations

import os
import warnings

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import nmsparse_op  # noqa: F401  (registers torch.ops.nmsparse.gemv)

DECODE_ONLY = os.environ.get("NM_DECODE_ONLY", "0") == "1"
WEIGHT_CPU = os.environ.get("NM_WEIGHT_CPU", "0") == "1" or DECODE_ONLY
SPARSE_BATCH = os.environ.get("NM_SPARSE_BATCH", "auto")
if SPARSE_BATCH not in ("auto", "0", "1"):
    raise ValueError(f"Unknown NM_SPARSE_BATCH={SPARSE_BATCH!r}; use auto, 0 or 1")
SPARSE_BATCH_MAX_ROWS = 128
SYNTH_INIT = os.environ.get("NM_SYNTH_INIT", "reference")
if SYNTH_INIT not in ("reference", "device"):
    raise ValueError(f"Unknown NM_SYNTH_INIT={SYNTH_INIT!r}; use 'reference' or 'device'")


def _bank_patterns(gen: torch.Generator, banks: int, M: int, nnz: int) -> torch.Tensor:
    """One sorted draw of nnz distinct positions out of M per bank, in bank order."""
    rows = [torch.randperm(M, generator=gen)[:nnz].sort().values for _ in range(banks)]
    if not rows:
        return torch.empty(0, nnz, dtype=torch.uint8)
    return torch.stack(rows).to(torch.uint8)


def _make_sparse(K, N, M, seed, device, init=None):
    """Synthetic packed weights for an N-output, K-input Linear at 50% N:M.

    Returns (mat_data [w, N] fp16, mat_index [K/M, M/2] uint8, w, nnz) on
    `device`. With the default init the values are bit-exact with the
    reference: the same CPU generator consumed by the same calls in the same
    order (fp32 normal draws scaled by 1/sqrt(K) then rounded to fp16, then one
    sorted randperm prefix per bank).
    """
    init = SYNTH_INIT if init is None else init
    nnz = M // 2
    banks = K // M
    w = banks * nnz
    if init == "device" and device != "cpu":
        gen = torch.Generator(device=device).manual_seed(seed)
        mat_data = (torch.randn(w, N, generator=gen, dtype=torch.float32, device=device) / (K ** 0.5)).to(
            torch.float16)
        keys = torch.rand(banks, M, generator=gen, device=device)
        mat_index = keys.argsort(dim=1)[:, :nnz].sort(dim=1).values.to(torch.uint8).contiguous()
        return mat_data, mat_index, w, nnz
    gen = torch.Generator().manual_seed(seed)
    scaled = torch.randn(w, N, generator=gen, dtype=torch.float32) / (K ** 0.5)
    mat_data = scaled.to(torch.float16)
    mat_index = _bank_patterns(gen, banks, M, nnz)
    if device != "cpu":
        mat_data = mat_data.to(device)
        mat_index = mat_index.to(device)
    return mat_data, mat_index, w, nnz


def pack_dense(weight: torch.Tensor, mat_index: torch.Tensor, M: int) -> torch.Tensor:
    """Packed [w, N] buffer of a dense [N, K] weight under a shared N:M pattern.

    mat_index is [K/M, nnz] (sorted in-group positions); mat_data[c, :] =
    weight[:, (c // nnz) * M + mat_index.flat[c]]. A pure gather (bit-exact);
    entries of `weight` outside the pattern are ignored.
    """
    N, K = weight.shape
    banks, nnz = mat_index.shape
    if banks * M != K:
        raise ValueError(f"mat_index has {banks} banks of M={M}, weight has K={K}")
    pos = (torch.arange(banks * nnz, device=mat_index.device) // nnz) * M + mat_index.reshape(-1).long()
    return weight[:, pos.to(weight.device)].t().contiguous()


def index_from_pruned(weight: torch.Tensor, M: int, nnz: int | None = None) -> torch.Tensor:
    """Shared N:M pattern [K/M, nnz] (sorted uint8 positions) of a dense [N, K]
    weight pruned with one mask for all N output rows.

    A position is kept when any row is non-zero there. A group with fewer than
    nnz such positions (kept weights that happen to be zero in every row) is
    completed with its lowest all-zero positions, which pack to zeros, so the
    packed weight still reproduces `weight` exactly. A group with more than
    nnz non-zero positions is not N:M with a shared mask: ValueError.
    """
    N, K = weight.shape
    nnz = M // 2 if nnz is None else nnz
    if K % M or not 0 < nnz <= M:
        raise ValueError(f"need K % M == 0 and 0 < nnz <= M; got K={K}, M={M}, nnz={nnz}")
    used = (weight != 0).any(dim=0).view(K // M, M)
    count = used.sum(dim=1)
    if bool((count > nnz).any()):
        g = int(torch.nonzero(count > nnz)[0, 0])
        raise ValueError(f"group {g} has {int(count[g])} non-zero positions, more than nnz={nnz}: the weight is "
                         f"not {nnz}:{M} sparse with a shared mask")
    # kept positions first (in ascending order), then the lowest unused ones
    key = (~used).to(torch.int64) * M + torch.arange(M, device=weight.device)
    pos = key.argsort(dim=1)[:, :nnz].sort(dim=1).values
    return pos.to(torch.uint8).contiguous()


class NmSparseLinear(nn.Module):
    """Linear layer whose decode path is the N:M sparse GEMV.

    N is the number of outputs (h), K the number of inputs, M the group size
    (50% sparsity: M/2 kept per group). Asserts K % M == 0 and N % 128 == 0 as
    the reference does (src/spmv/nmsparse_linear.py:39).
    """

    def __init__(self, N, K, M, seed, device, dense_weight=None, *, init=None):
        super().__init__()
        assert K % M == 0 and N % 128 == 0, (K, N, M)
        self._weight_cpu = None
        self.weight = None
        if dense_weight is not None:
            if WEIGHT_CPU:
                self._weight_cpu = dense_weight.detach().cpu()
                del dense_weight
                if device != "cpu":
                    torch.cuda.empty_cache()
            else:
                self.weight = dense_weight
        md, mi, w, nnz = _make_sparse(K, N, M, seed, device, init=init)
        self.register_buffer("mat_data", md)
        self.register_buffer("mat_index", mi)
        self.h, self.w, self.block_width, self.vec_width = N, w, nnz, M

    @classmethod
    def from_dense(cls, weight: torch.Tensor, mat_index: torch.Tensor, M: int, keep_dense: bool = False):
        """Build from a real dense [N, K] weight and its shared N:M pattern
        (mat_index [K/M, M/2] uint8). `keep_dense` keeps `weight` for prefill."""
        N, K = weight.shape
        if K % M or N % 128 or mat_index.shape != (K // M, M // 2):
            raise ValueError(f"need K % M == 0, N % 128 == 0 and mat_index [K/M, M/2]; got N={N}, K={K}, M={M}, "
                             f"mat_index {tuple(mat_index.shape)}")
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self._weight_cpu = None
        self.weight = weight if keep_dense else None
        mi = mat_index.to(device=weight.device, dtype=torch.uint8).contiguous()
        self.register_buffer("mat_data", pack_dense(weight, mi, M).to(torch.float16))
        self.register_buffer("mat_index", mi)
        self.h, self.w, self.block_width, self.vec_width = N, (K // M) * (M // 2), M // 2, M
        return self

    @classmethod
    def from_pruned(cls, weight: torch.Tensor, M: int, keep_dense: bool = False):
        """Build from a dense [N, K] weight already pruned to 50% N:M with one
        mask shared by all rows (the mask is recovered by index_from_pruned)."""
        return cls.from_dense(weight, index_from_pruned(weight, M), M, keep_dense=keep_dense)

    @classmethod
    def empty(cls, N: int, K: int, M: int, device, dtype=torch.float16):
        """Module with uninitialised packed buffers of the right shapes, to be
        filled by load_state_dict (e.g. from a saved compressed checkpoint)."""
        if K % M or N % 128:
            raise ValueError(f"need K % M == 0 and N % 128 == 0; got N={N}, K={K}, M={M}")
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self._weight_cpu = None
        self.weight = None
        nnz, banks = M // 2, K // M
        self.register_buffer("mat_data", torch.empty(banks * nnz, N, dtype=dtype, device=device))
        self.register_buffer("mat_index", torch.zeros(banks, nnz, dtype=torch.uint8, device=device))
        self.h, self.w, self.block_width, self.vec_width = N, banks * nnz, nnz, M
        return self

    def to_dense(self, dtype=None) -> torch.Tensor:
        """The dense [N, K] weight this module computes with: the packed weights
        scattered back to their input columns, zeros elsewhere (the inverse of
        pack_dense, a pure scatter: bit-exact). `dtype` converts the result."""
        banks, nnz = self.mat_index.shape
        K = banks * self.vec_width
        pos = (torch.arange(banks * nnz, device=self.mat_index.device) // nnz) * self.vec_width \
            + self.mat_index.reshape(-1).long()
        dense = torch.zeros(self.h, K, dtype=dtype or self.mat_data.dtype, device=self.mat_data.device)
        dense[:, pos.to(dense.device)] = self.mat_data.t().to(dense.dtype)
        return dense

    def _prefill_weight(self, device):
        if self.weight is not None:
            return self.weight
        if self._weight_cpu is None:
            raise RuntimeError("prefill requires dense weight")
        return self._weight_cpu.to(device)

    def _has_dense(self) -> bool:
        return self.weight is not None or self._weight_cpu is not None

    def forward(self, x):
        rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
        args = (self.mat_data, self.mat_index, self.w, self.h, self.block_width, self.vec_width)
        if SPARSE_BATCH != "0" and rows > 1:
            if not self._has_dense() or (SPARSE_BATCH == "1" and rows <= SPARSE_BATCH_MAX_ROWS):
                group = self.__dict__.get("_siblings")
                if group is not None and not torch.compiler.is_compiling():
                    y = group.output(self, x)
                    if y is not None:
                        return y
                return torch.ops.nmsparse.spmm(x, *args)
        if x.shape[-2] == 1:
            group = self.__dict__.get("_siblings")
            if group is not None and not torch.compiler.is_compiling():
                y = group.output(self, x)
                if y is not None:
                    return y
            return torch.ops.nmsparse.gemv(x, *args)
        return F.linear(x, self._prefill_weight(x.device))

    def extra_repr(self) -> str:
        return f"h={self.h}, w={self.w}, N:M={self.block_width}:{self.vec_width}"


class SiblingLaunch:
    """Sparse Linears of one block that read the same input (q/k/v, gate/up),
    computed by one grouped launch (hip_spmv.nmsparse_gemv_grouped) instead of
    one launch each, without any change to the model code that calls them.

    The first member called with a one-row input launches the grouped GEMV for
    every member (with 9-128 rows of fp16 / bf16 on the sparse path: the
    grouped matrix-core SpMM, hip_spmv.nmsparse_spmm_group_hip) and keeps the
    other members' outputs; a member then called with the very same input
    tensor (same object, unchanged version counter) takes its output, once.
    Any other call (another input, a repeated member, other row counts, a
    dtype or device the grouped launch does not take, or torch.compile
    tracing) goes through the member's own op as before, so the results never
    depend on the call order, only the last bit of a sum may (the grouped plan
    splits the columns like a launch of the summed width).
    The bookkeeping is on the host, so under hipGraph capture the graph holds
    the one grouped launch and the siblings read its outputs. The group holds
    the input tensor it launched for until the next launch, so that tensor's
    memory cannot be reused under it. No reference counterpart: the reference
    launches every Linear on its own (src/spmv/nmsparse_linear.py:62-68).

    Inference tensors (created under torch.inference_mode(), as the
    reference's benchmarks run: benchmarks/bench_llama_3_8b_fp16_fixed_ptx.py:87)
    carry no version counter, so for them "the very same input" means the same
    tensor object only: an in-place change of that tensor between two
    members' calls is not seen (the later member gets the output computed
    before the change). Model code that modifies a Linear's input in place
    between its siblings' calls should untie them (untie_siblings).

    When a launch leaves outputs that no member claims before the next launch
    (siblings fed different inputs, e.g. cross-attention's q from the decoder
    and k/v from the encoder), the grouped launch streamed those members'
    weights for nothing; the group warns once (RuntimeWarning) and keeps
    serving calls, so results are unaffected.
    """

    def __init__(self, members):
        if not 2 <= len(members) <= 4:
            raise ValueError("a sibling group takes 2 to 4 Linears")
        m0 = members[0]
        for m in members:
            if not isinstance(m, NmSparseLinear) or (m.w, m.block_width, m.vec_width) != (
                    m0.w, m0.block_width, m0.vec_width):
                raise ValueError("siblings must be NmSparseLinear with the same K and N:M")
        self.members = list(members)
        self._x = None
        self._version = -1
        self._pending = {}
        self._warned = False

    def _usable(self, x) -> bool:
        md = self.members[0].mat_data
        rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
        grouped_rows = rows == 1 or (x.dtype in (torch.float16, torch.bfloat16) and 8 < rows <= 128)
        return (x.is_cuda and x.dtype == md.dtype and x.device == md.device and x.is_contiguous() and grouped_rows
                and all(m.mat_data.device == md.device for m in self.members))

    def output(self, member, x):
        """member(x) from the group's launch, or None when the group does not
        serve this call (the member then launches on its own)."""
        if not self._usable(x):
            return None
        i = next(j for j, m in enumerate(self.members) if m is member)
        version = None if x.is_inference() else x._version  # inference tensors have no version counter
        if self._x is x and self._version == version and i in self._pending:
            return self._pending.pop(i)
        if self._pending and not self._warned:
            self._warned = True
            names = ", ".join(str(j) for j in sorted(self._pending))
            warnings.warn(
                f"nmsparse: a SiblingLaunch of {len(self.members)} Linears launched again while member(s) {names} "
                "had not taken their outputs of its previous launch (siblings called with different inputs?); "
                "those weights were streamed for nothing. Results are unaffected; untie_siblings(model) makes "
                "every Linear launch on its own.", RuntimeWarning, stacklevel=3)
        from .hip_spmv import nmsparse_gemv_grouped, nmsparse_spmm_group_hip

        m0 = self.members[0]
        outs = [torch.empty(*x.shape[:-1], m.h, dtype=x.dtype, device=x.device) for m in self.members]
        mats = [(m.mat_data, m.mat_index) for m in self.members]
        if x.numel() == x.shape[-1]:
            nmsparse_gemv_grouped(x.view(1, -1), mats, m0.block_width, m0.vec_width, outs=[o.view(1, -1) for o in outs])
        else:
            nmsparse_spmm_group_hip(x, mats, m0.block_width, m0.vec_width, outs=outs)
        self._x, self._version = x, version
        self._pending = {j: o for j, o in enumerate(outs) if j != i}
        return outs[i]


def tie_siblings(*members) -> SiblingLaunch:
    """Make `members` (NmSparseLinear of one block reading the same input) one
    SiblingLaunch; returns it. Replaces any group they were in."""
    group = SiblingLaunch(members)
    for m in members:
        m.__dict__["_siblings"] = group  # a plain attribute: not a submodule, not in the state_dict
    return group


def untie_siblings(model) -> int:
    """Drop every sibling group in `model` (each Linear launches on its own
    again); returns the number of Linears untied."""
    n = 0
    for mod in model.modules():
        if mod.__dict__.pop("_siblings", None) is not None:
            n += 1
    return n


# Decoder-block layouts: (sub-module attribute, Linear names in swap order).
# gpt-fast fuses attention into wqkv/wo and names the MLP w1/w3/w2; Hugging
# Face decoder layers use self_attn.{q,k,v,o}_proj and mlp.{gate,up,down}_proj
# (src/spmv/nmsparse_linear.py:83-91).
_ATTENTION_LAYOUTS = (
    ("attention", ("wqkv", "wo")),
    ("self_attn", ("q_proj", "k_proj", "v_proj", "o_proj")),
)
_MLP_LAYOUTS = (
    ("feed_forward", ("w1", "w3", "w2")),
    ("mlp", ("gate_proj", "up_proj", "down_proj")),
)


# Linears of a layout that read the same input: tied by swap_to_nmsparse.
_SIBLINGS = {"wqkv": None, "q_proj": ("q_proj", "k_proj", "v_proj"), "w1": ("w1", "w3"),
             "gate_proj": ("gate_proj", "up_proj")}


def _resolve_layout(blk, layouts, kind):
    """The (sub-module, Linear names) of the first known layout `blk` has."""
    for attr, names in layouts:
        sub = getattr(blk, attr, None)
        if sub is not None:
            return sub, names
    known = ", ".join(f".{attr}" for attr, _ in layouts)
    raise AttributeError(
        f"decoder block {type(blk).__name__} has none of the known {kind} sub-modules ({known}); "
        "swap_to_nmsparse does not recognize this block's layout."
    )


def _swap_linears(submodule, names, M, device, seed, cnt, init=None, keep_dense=None, from_weights=False):
    """Replace submodule.<name> for each name, numbering seeds from seed + cnt."""
    keep = (not DECODE_ONLY) if keep_dense is None else keep_dense
    for name in names:
        old = getattr(submodule, name)
        N, K = old.weight.shape
        if from_weights:
            w = old.weight.detach().to(device)
            new = NmSparseLinear.from_pruned(w, M, keep_dense=keep)
        else:
            dense = old.weight if keep else None
            del old
            setattr(submodule, name, None)
            torch.cuda.empty_cache()
            new = NmSparseLinear(N, K, M, seed + cnt, device, dense_weight=dense, init=init)
        setattr(submodule, name, new)
        cnt += 1
    return cnt


def swap_to_nmsparse(model, M, device, seed=0, block_devices=None, *, init=None, keep_dense=None,
                     from_weights=False, tie=True):
    """Swap every attention and MLP Linear of `model.layers` to NmSparseLinear.

    Blocks are visited in order, attention before MLP, Linears in layout
    order; the j-th swapped Linear uses seed `seed + j`. `block_devices`
    optionally gives one device (index or "cuda:N") per block. Returns the
    number of swapped Linears. Keyword-only extras of this build: `init`
    ("reference" | "device", default from NM_SYNTH_INIT), `keep_dense`
    (default: not NM_DECODE_ONLY), `from_weights` (pack each Linear's own
    weight, which must already be 50% M-group pruned with a shared mask,
    instead of drawing synthetic weights; seeds are then unused) and `tie`
    (default True: the Linears of a block that read the same input, q/k/v
    and gate/up (w1/w3), become one SiblingLaunch, so the unchanged model
    code runs them as one grouped launch; untie_siblings undoes it).
    """
    cnt = 0
    for i, blk in enumerate(model.layers):
        blk_device = device
        if block_devices is not None:
            d = block_devices[i]
            blk_device = d if isinstance(d, str) else f"cuda:{d}"
        for layouts, kind in ((_ATTENTION_LAYOUTS, "attention"), (_MLP_LAYOUTS, "feed-forward")):
            sub, names = _resolve_layout(blk, layouts, kind)
            cnt = _swap_linears(sub, names, M, blk_device, seed, cnt, init, keep_dense, from_weights)
            sibs = _SIBLINGS.get(names[0])
            if tie and sibs:
                tie_siblings(*(getattr(sub, n) for n in sibs))
    return cnt


__all__ = ["NmSparseLinear", "swap_to_nmsparse", "pack_dense", "index_from_pruned", "_make_sparse", "SiblingLaunch",
           "tie_siblings", "untie_siblings"]
