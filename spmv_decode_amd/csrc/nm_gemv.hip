// nm_gemv.hip — host side of the shared-mask N:M sparse GEMV for MI355X:
// configuration metadata, launch planning (tiles, split-K, workspace layout),
// argument validation and the C ABI declared in include/nmsparse_hip.h. The
// kernels are in nm_gemv_kernel.h (instantiated by nm_gemv_inst.hip).

#include <mutex>

#include "nm_gemv_kernel.h"

namespace nm_hip {
namespace {

// ---------------------------------------------------------------------------
// Configuration tables (static; no runtime autotuning).
// ---------------------------------------------------------------------------
struct Config {
  int th;       // lanes along the output rows (tile = 8*th rows)
  int u;        // rows per lane per chunk
  bool nt;      // non-temporal weight loads
};

#define NM_META(TH, U, NT) {TH, U, NT},
const Config kConfigs[kNumConfigs] = {NM_PLAIN_CONFIGS(NM_META)};
const Config kDualConfigs[kNumDualConfigs] = {NM_PAIR_CONFIGS(NM_META)};
#undef NM_META

const KernelRow* kernel_table(int dtype, bool pair) {
  switch (dtype) {
    case NM_DTYPE_F16: return pair ? kPairKernelsF16 : kPlainKernelsF16;
    case NM_DTYPE_BF16: return pair ? kPairKernelsBF16 : kPlainKernelsBF16;
    default: return pair ? kPairKernelsF32 : kPlainKernelsF32;
  }
}

inline int gather_slot(int rows) {
  return rows <= kBlock ? 0 : (rows <= 2 * kBlock ? 1 : (rows <= 4 * kBlock ? 2 : 3));
}

struct Plan {
  int cfg;
  int splits;
  int rows_per_split;
  int nprob;
  int tiles[kMaxProblems];
  int block_begin[kMaxProblems];
  int blocks;
  size_t ticket_off[kMaxProblems];   // in uint32 units from the workspace start
  size_t partial_off[kMaxProblems];  // in bytes from the workspace start
  size_t ssq_off;                    // carried input: per-workgroup ssq slots, bytes from the start
  size_t workspace;
};

inline int ceil_div(long long a, long long b) { return (int)((a + b - 1) / b); }

int validate_shape(int h, int w, int nnz, int m) {
  if (h <= 0 || w <= 0 || nnz <= 0 || m <= 0 || m > 256 || nnz > m) return NM_ERR_BAD_SHAPE;
  if (h % 128 != 0) return NM_ERR_H_NOT_MULTIPLE_128;
  if (w % nnz != 0) return NM_ERR_W_NOT_MULTIPLE_NNZ;
  const long long K = (long long)(w / nnz) * (long long)m;
  if (K > 0x7fffffffLL) return NM_ERR_BAD_SHAPE;
  return NM_OK;
}

// The library's own choice of configuration and split count, from hipGraph
// sweeps of the decoder's launches on MI355X at the Llama-3.1-8B, Qwen3-14B and
// Qwen3-32B shapes (h_total: summed output width of the launch). Single
// matrix: 128-row tiles up to 4096 outputs, 256-row tiles up to 16384,
// 512-row tiles beyond. Gate/up pair: 256-row tiles with 32-row chunks up to
// 14336 outputs, 512-row tiles with 32-row chunks beyond; with a carried
// input, 512-row tiles with 16-row chunks (half the workgroups of 256-row
// tiles, so half the carried partials read: 23.0 against 24.3 us at the
// Llama-3.1-8B shape).
int auto_config(long long h_total, int nmat, bool carried) {
  if (nmat == 2) return carried ? 4 : (h_total > 14336 ? 5 : 1);
  return h_total > 16384 ? 6 : (h_total > 4096 ? 3 : 1);
}

// Workgroups that run at once, one per CU: an MI355X has 256 CUs. The split
// count below is chosen for this many; it changes speed only, never results.
constexpr int kPlanCUs = 256;

// Default split count. About 8 splits of the compressed columns per tile: the
// cost of a split-K handoff (one partial publish, one arrival atomic on a
// per-tile counter, one reduction) grows with the split count faster than
// the extra parallelism pays back. Two corrections from the sweeps:
//  * a single matrix with long columns (w >= 6144) and few tiles takes up to
//    12 splits while the grid still fits one workgroup per CU;
//  * a grid of more workgroups than CUs whose last round is mostly empty
//    (e.g. 320 = 1.25 rounds) waits for the few CUs that run two: then the
//    split count in 9..12 whose rounds are fullest is taken, or, when none
//    fills 80% of its last round, the one in 4..12 that does best.
// `eff(s)` is the number of splits a request for s splits gets once the rows
// per split are rounded to whole chunks.
//  * a gate/up pair of 512-row tiles (a carried input, or wider than 14336
//    outputs) takes one round of workgroups: the largest split count whose
//    grid has at most 7/8 of the CUs' workgroups, else the smallest grid of
//    at most one per CU (sweeps: a second round of a few workgroups costs
//    4-9 us; Qwen3-14B 33.1 us at 6 splits against 34.5 at 7, Qwen3-32B 44.1
//    at 4 against 46.6 at 10).
template <class EffSplits>
int auto_splits(int tiles, int w, int nmat, EffSplits eff, bool one_round) {
  if (one_round) {
    for (int s = 16; s >= 2; --s)
      if ((long long)tiles * eff(s) <= kPlanCUs * 7 / 8) return s;
    int best = 0;
    long long fewest = kPlanCUs + 1;
    for (int s = 2; s <= 16; ++s) {
      const long long blocks = (long long)tiles * eff(s);
      if (blocks < fewest) {
        fewest = blocks;
        best = s;
      }
    }
    if (best) return best;
  }
  auto balance = [&](int s) {
    const double rounds = (double)tiles * eff(s) / kPlanCUs;
    return rounds <= 1.0 ? 1.0 : rounds / ceil(rounds);
  };
  if (nmat == 1 && w >= 6144) {
    for (int s = 12; s >= 8; --s)
      if ((long long)tiles * eff(s) <= kPlanCUs) return s;
  }
  int best = 8;
  double best_balance = balance(8);
  if (best_balance >= 0.8) return best;
  auto consider = [&](int s) {
    const double b = balance(s);
    if (b > best_balance + 1e-9) {
      best = s;
      best_balance = b;
    }
  };
  for (int s = 9; s <= 12; ++s) consider(s);  // ties keep the smaller count
  if (best_balance >= 0.8) return best;
  for (int s = 7; s >= 4; --s) consider(s);   // ties keep the larger count
  return best;
}

// Plan a launch of `nprob` problems (widths hs[]) sharing w, nnz, m, with
// `nmat` matrices per workgroup. The workspace holds the counters of every
// problem in its first NM_TICKET_BYTES and then nmat * splits * h floats of
// partial sums per problem.
int make_plan(int nprob, const int* hs, int w, int nnz, int m, int nmat, int cfg, int splits, Plan* p,
              int max_rows = kMaxRows, int batch = 1, int row_align = 1, bool carried = false) {
  if (nprob < 1 || nprob > kMaxProblems || (nmat == 2 && nprob != 1)) return NM_ERR_BAD_SHAPE;
  long long h_total = 0;
  for (int i = 0; i < nprob; ++i) {
    const int rc = validate_shape(hs[i], w, nnz, m);
    if (rc != NM_OK) return rc;
    h_total += hs[i];
  }
  const int ncfg = nmat == 2 ? kNumDualConfigs : kNumConfigs;
  if (cfg < 0) cfg = auto_config(h_total, nmat, carried);
  if (cfg >= ncfg) return NM_ERR_BAD_CONFIG;
  const Config& c = nmat == 2 ? kDualConfigs[cfg] : kConfigs[cfg];
  const int HT = c.th * kVec;
  const int CH = (kBlock / c.th) * c.u;
  // Rows per split: whole chunks, and whole multiples of row_align (a carried
  // input needs whole groups of nnz columns per split).
  int AL = CH;
  while (AL % row_align != 0) AL += CH;
  auto rows_for = [&](int s) {
    if (s > w) s = w;
    int r = ceil_div(ceil_div(w, s), AL) * AL;
    if (r > max_rows) r = max_rows >= AL ? (max_rows / AL) * AL : AL;
    return r < AL ? AL : r;
  };
  if (splits <= 0) {
    int tiles = 0;
    for (int i = 0; i < nprob; ++i) tiles += ceil_div(hs[i], HT);
    const bool one_round = nmat == 2 && c.th == 64 && (carried || h_total > 14336);
    splits = auto_splits(tiles, w, nmat, [&](int s) { return ceil_div(w, rows_for(s)); }, one_round);
  }
  const int rows = rows_for(splits);
  splits = ceil_div(w, rows);
  p->cfg = cfg;
  p->ssq_off = 0;
  p->splits = splits;
  p->rows_per_split = rows;
  p->nprob = nprob;
  long long blocks = 0;
  size_t tickets = 0;
  size_t bytes = NM_TICKET_BYTES;
  for (int i = 0; i < nprob; ++i) {
    p->tiles[i] = ceil_div(hs[i], HT);
    p->block_begin[i] = (int)blocks;
    blocks += (long long)p->tiles[i] * (long long)splits;
    p->ticket_off[i] = tickets;
    tickets += (size_t)p->tiles[i];
    p->partial_off[i] = bytes;
    if (splits > 1) bytes += (size_t)nmat * (size_t)batch * (size_t)splits * (size_t)hs[i] * sizeof(float);
  }
  if (tickets > (size_t)kMaxTickets || blocks > 0x7fffffffLL) return NM_ERR_BAD_SHAPE;
  p->blocks = (int)blocks;
  p->workspace = bytes;
  return NM_OK;
}

// The plan of a launch described by `d`. A producer (carry_out: one GEMV whose
// split-K reduction moves into the next launch) has no handoff, so more
// splits cost it only the partials its consumer reads: where the default plan
// would leave a quarter of the CUs or more idle (the Qwen3-14B / Qwen3-32B
// o_proj: 20 tiles of 256 rows x 8 splits, 160 workgroups), it takes 128-row
// tiles and the most splits (<= kMaxCarry) that fit one workgroup per CU
// (sweeps: 7.13 -> 6.52 us and 9.28 -> 8.81 us, its consumer then reading 5
// or 6 splits instead of 8). A consumer's plan puts whole groups of columns,
// at most 512, in each split (the carried-input kernels cover gather slots 0
// and 1).
constexpr int kProducerConfig = 1;  // th16_u8: 128-row tiles, 128-row chunks

int plan_desc(const nm_gemv_launch_desc& d, int nprob, const int* hs, int nmat, Plan* p) {
  const bool carry_in = d.carry_in != nullptr;
  int rc = make_plan(nprob, hs, d.w, d.nnz, d.m, nmat, d.config_id, d.splits, p, carry_in ? 2 * kBlock : kMaxRows,
                     1, carry_in ? d.nnz : 1, carry_in);
  const bool producer = d.carry_out != nullptr && nmat == 1 && nprob == 1 && !carry_in;
  if (rc != NM_OK || !producer || d.config_id >= 0 || d.splits > 0 || p->blocks > kPlanCUs * 3 / 4) return rc;
  for (int s = kMaxCarry; s >= 2; --s) {
    Plan q;
    if (make_plan(1, hs, d.w, d.nnz, d.m, 1, kProducerConfig, s, &q) == NM_OK && q.splits <= kMaxCarry &&
        q.blocks <= kPlanCUs) {
      if (q.blocks > p->blocks) *p = q;
      break;
    }
  }
  return NM_OK;
}

// Whether [ptr, ptr + bytes) overlaps a buffer the launch described by `d`
// reads or writes other than vec (norm weight, matrices and indices,
// outputs, residuals, head norms, RoPE table, position, workspace, carried
// input and output, SiLU-product input, vec_out, zero_buf), leaving out the
// descriptor field `self` (the buffer being checked: &d.vec_out, &d.zero_buf
// or &d.silu_in).
bool overlaps_launch(const nm_gemv_launch_desc& d, int nprob, int K, size_t esize, const void* workspace,
                     size_t workspace_bytes, int splits, const void* self, const void* ptr, size_t bytes) {
  const uintptr_t v0 = (uintptr_t)ptr;
  auto clash_field = [&](const void* field, const void* other, size_t n) {
    const uintptr_t b = (uintptr_t)other;
    return field != self && other != nullptr && n > 0 && v0 < b + n && b < v0 + bytes;
  };
  auto clash = [&](const void* other, size_t n) { return clash_field(nullptr, other, n); };
  const size_t slice_k = (size_t)K * esize;
  const size_t rope_bytes = (size_t)(d.pos_limit > 0 ? d.pos_limit : 0) * (size_t)(d.head_dim / 2) * 2 * sizeof(float);
  if (clash(d.carry_in, (size_t)d.carry_splits * (size_t)K * sizeof(float)) || clash(d.norm_weight, slice_k) ||
      clash(workspace, workspace_bytes) || clash(d.pos, sizeof(long long)) || clash(d.rope_table, rope_bytes) ||
      clash_field(&d.vec_out, d.vec_out, slice_k) ||
      clash_field(&d.zero_buf, d.zero_buf, (size_t)(d.zero_len > 0 ? d.zero_len : 0) * sizeof(float)) ||
      clash_field(&d.silu_in, d.silu_in,
                  (size_t)(2 * (size_t)K + (size_t)(d.silu_ssq_n > 0 ? d.silu_ssq_n : 0)) * sizeof(float)))
    return true;
  for (int i = 0; i < d.nprob; ++i) {
    const nm_gemv_problem& q = d.prob[i];
    if (clash(q.mat_data, (size_t)d.w * (size_t)q.h * esize) || clash(q.mat_index, (size_t)d.w)) return true;
  }
  const bool pair = d.kind == NM_KIND_GATE_UP;
  if (d.carry_out) {  // a producer writes its partials (an accumulating one a row, the pair 2h + 16 floats)
    const size_t n = pair ? 2 * (size_t)d.prob[0].h + 16 : (size_t)(d.carry_accumulate ? 1 : splits) * (size_t)d.prob[0].h;
    if (clash(d.carry_out, n * sizeof(float))) return true;
  }
  for (int i = 0; i < nprob; ++i) {
    const nm_gemv_problem& q = d.prob[i];
    size_t out_elems = (size_t)q.h;
    if (q.head_stride != 0 || q.elem_stride != 0 || q.pos_stride != 0) {
      const long long hd = d.head_dim > 0 ? d.head_dim : 1;
      out_elems = (size_t)((q.h / hd - 1) * q.head_stride + (hd - 1) * q.elem_stride +
                           (long long)(d.pos_limit > 1 ? d.pos_limit - 1 : 0) * q.pos_stride + 1);
    }
    if ((!d.carry_out && clash(q.out, out_elems * esize)) || clash(q.residual, (size_t)q.h * esize) ||
        clash(q.head_norm, (size_t)(d.head_dim > 0 ? d.head_dim : 0) * esize))
      return true;
  }
  return false;
}

// Validate a launch descriptor, plan it and launch. Every entry point of the
// C ABI goes through here. With `workspace_needed` it only plans (and reports
// the workspace size); with `validate_only` it runs every check and returns
// before launching.
int launch(const nm_gemv_launch_desc& d, void* workspace, size_t workspace_bytes, void* stream,
           size_t* workspace_needed, bool validate_only = false) {
  if (d.dtype < NM_DTYPE_F16 || d.dtype > NM_DTYPE_F32) return NM_ERR_BAD_CONFIG;
  if (d.kind != NM_KIND_GROUPED && d.kind != NM_KIND_GATE_UP) return NM_ERR_BAD_CONFIG;
  const bool pair = d.kind == NM_KIND_GATE_UP;
  const int nmat = pair ? 2 : 1;
  const int nprob = pair ? 1 : d.nprob;  // output problems
  if (pair ? d.nprob != 2 : (d.nprob < 1 || d.nprob > kMaxProblems)) return NM_ERR_BAD_SHAPE;
  int hs[kMaxProblems];
  for (int i = 0; i < nprob; ++i) hs[i] = d.prob[i].h;
  if (pair && d.prob[1].h != d.prob[0].h) return NM_ERR_BAD_SHAPE;
  const bool carry_in = d.carry_in != nullptr;
  const bool carry_out = d.carry_out != nullptr;
  const bool silu_in = d.silu_in != nullptr;
  // a carried input and a producer at once: only the accumulating gate/up pair
  if (carry_in && carry_out && !(pair && d.carry_accumulate)) return NM_ERR_BAD_EPILOGUE;
  if (d.carry_accumulate && !carry_out) return NM_ERR_BAD_EPILOGUE;
  if (pair && carry_out && !d.carry_accumulate) return NM_ERR_BAD_EPILOGUE;  // the pair's only producer form
  if (d.nnz <= 0) return NM_ERR_BAD_SHAPE;
  Plan p;
  int rc = plan_desc(d, nprob, hs, nmat, &p);
  if (rc != NM_OK) return rc;
  // the accumulating pair with a carried input stores one sum of squares per
  // split in the 16 slots after its sums
  if (pair && carry_out && carry_in && p.splits > 16) return NM_ERR_BAD_EPILOGUE;
  if (carry_in) {
    // The ssq slots follow the partials: one float per workgroup.
    p.workspace = (p.workspace + 255) & ~(size_t)255;
    p.ssq_off = p.workspace;
    if (p.splits > 1) p.workspace += (size_t)p.blocks * sizeof(float);
  }
  if (workspace_needed) {
    *workspace_needed = p.workspace;
    return NM_OK;
  }
  if ((!d.vec && !silu_in) || !workspace) return NM_ERR_NULL_POINTER;
  for (int i = 0; i < d.nprob; ++i)
    if (!d.prob[i].mat_data || !d.prob[i].mat_index) return NM_ERR_NULL_POINTER;
  for (int i = 0; i < nprob; ++i)
    if (!d.prob[i].out && !carry_out) return NM_ERR_NULL_POINTER;
  if (d.vec_stride < 1) return NM_ERR_BAD_SHAPE;
  for (int i = 0; i < d.nprob; ++i)
    if (((uintptr_t)d.prob[i].mat_data & 15u) != 0) return NM_ERR_MISALIGNED;
  for (int i = 0; i < nprob; ++i)
    if (!carry_out && ((uintptr_t)d.prob[i].out & 15u) != 0) return NM_ERR_MISALIGNED;
  if (((uintptr_t)workspace & 255u) != 0) return NM_ERR_MISALIGNED;
  if (workspace_bytes < p.workspace) return NM_ERR_WORKSPACE;

  // Epilogue / prologue arguments.
  const int K = (d.w / d.nnz) * d.m;
  const size_t esize = d.dtype == NM_DTYPE_F32 ? 4 : 2;
  if (d.norm_weight) {
    if (!(d.norm_eps >= 0.0f) || d.vec_stride != 1 || ((uintptr_t)d.vec & 15u) != 0 ||
        ((size_t)K * esize) % 16 != 0)
      return NM_ERR_BAD_EPILOGUE;
  }
  const Config& c = pair ? kDualConfigs[p.cfg] : kConfigs[p.cfg];
  const int HT = c.th * kVec;
  bool any_pos = false, any_rope = false;
  for (int i = 0; i < nprob; ++i) {
    const nm_gemv_problem& q = d.prob[i];
    const bool layout = q.head_stride != 0 || q.elem_stride != 0 || q.pos_stride != 0;
    const bool heads = q.head_norm != nullptr || q.rope != 0 || layout;
    if (!heads) continue;
    if (pair) return NM_ERR_BAD_EPILOGUE;  // the pair writes a plain [h] output
    if (d.head_dim <= 0 || d.head_dim % 64 != 0 || q.h % d.head_dim != 0 || HT % d.head_dim != 0)
      return NM_ERR_BAD_EPILOGUE;
    if (q.head_norm && !(d.head_norm_eps >= 0.0f)) return NM_ERR_BAD_EPILOGUE;
    any_pos = any_pos || q.rope != 0 || q.pos_stride != 0;
    any_rope = any_rope || q.rope != 0;
  }
  if (any_pos && (!d.pos || d.pos_limit <= 0)) return NM_ERR_BAD_EPILOGUE;
  if (any_rope && !d.rope_table) return NM_ERR_BAD_EPILOGUE;
  if (carry_out) {
    const nm_gemv_problem& q = d.prob[0];
    if (pair) {
      // the accumulating pair: raw sums and the norm's sum of squares go to the consumer
      if (q.residual) return NM_ERR_BAD_EPILOGUE;
    } else if (d.nprob != 1 || d.norm_weight || q.residual || q.head_norm || q.rope || q.head_stride ||
               q.elem_stride || q.pos_stride) {
      return NM_ERR_BAD_EPILOGUE;  // one plain GEMV: its epilogue moves into the consumer
    }
    if (((uintptr_t)d.carry_out & 15u) != 0) return NM_ERR_MISALIGNED;
  }
  if (silu_in) {
    const nm_gemv_problem& q = d.prob[0];
    if (pair || d.nprob != 1 || d.norm_weight || carry_in || q.head_norm || q.rope || q.head_stride ||
        q.elem_stride || q.pos_stride || d.silu_ssq_n < 0 || d.silu_ssq_n > 16 ||
        (d.silu_ssq_n > 0 && d.silu_k <= 0) || !(d.silu_eps >= 0.0f))
      return NM_ERR_BAD_EPILOGUE;
    if (((uintptr_t)d.silu_in & 15u) != 0) return NM_ERR_MISALIGNED;
    // every workgroup gathers from silu_in while others write the launch's
    // outputs (or add into carry_out): it must overlap none of them
    if (overlaps_launch(d, nprob, K, esize, workspace, workspace_bytes, p.splits, &d.silu_in, d.silu_in,
                        (2 * (size_t)K + (size_t)d.silu_ssq_n) * sizeof(float)))
      return NM_ERR_BAD_EPILOGUE;
  }
  if (d.zero_buf) {
    if (d.zero_len <= 0 || d.zero_len % 4 != 0) return NM_ERR_BAD_EPILOGUE;
    if (((uintptr_t)d.zero_buf & 15u) != 0) return NM_ERR_MISALIGNED;
  }
  if (carry_in) {
    if (!d.norm_weight || !d.vec_out) return NM_ERR_BAD_EPILOGUE;
    if (d.carry_splits < 1 || d.carry_splits > kMaxCarry || d.m % 4 != 0) return NM_ERR_BAD_EPILOGUE;
    if (p.rows_per_split % d.nnz != 0 || gather_slot(p.rows_per_split) > 1) return NM_ERR_BAD_EPILOGUE;
    const long long slice = (long long)(p.rows_per_split / d.nnz) * d.m;  // K positions a split reads
    if (slice > 4 * kBlock) return NM_ERR_BAD_EPILOGUE;
    if (((uintptr_t)d.carry_in & 15u) != 0 || ((uintptr_t)d.vec_out & 15u) != 0 ||
        ((uintptr_t)d.norm_weight & 15u) != 0)
      return NM_ERR_MISALIGNED;
    const uintptr_t vo = (uintptr_t)d.vec_out, vi = (uintptr_t)d.vec;
    if (vo < vi + (size_t)K * esize && vi < vo + (size_t)K * esize) return NM_ERR_BAD_EPILOGUE;  // overlap
    // Tile 0's workgroups write vec_out while the other workgroups still read
    // every input of the launch and write its outputs: vec_out must overlap
    // none of them.
    if (overlaps_launch(d, nprob, K, esize, workspace, workspace_bytes, p.splits, &d.vec_out, d.vec_out,
                        (size_t)K * esize))
      return NM_ERR_BAD_EPILOGUE;
  }
  // The buffer this launch clears must not be one it reads or writes.
  if (d.zero_buf && ((d.vec && (uintptr_t)d.zero_buf < (uintptr_t)d.vec + (size_t)K * esize &&
                      (uintptr_t)d.vec < (uintptr_t)d.zero_buf + (size_t)d.zero_len * 4) ||
                     overlaps_launch(d, nprob, K, esize, workspace, workspace_bytes, p.splits, &d.zero_buf, d.zero_buf,
                                     (size_t)d.zero_len * sizeof(float))))
    return NM_ERR_BAD_EPILOGUE;
  if (validate_only) return NM_OK;

  Args a;
  memset(&a, 0, sizeof(a));
  a.vec = d.vec;
  a.vec_stride = d.vec_stride;
  a.norm_w = d.norm_weight;
  a.norm_eps = d.norm_eps;
  a.head_eps = d.head_norm_eps;
  a.head_dim = d.head_dim;
  a.pos = d.pos;
  a.pos_limit = d.pos_limit;
  a.rope = reinterpret_cast<const float2*>(d.rope_table);
  a.w = d.w;
  a.nnz = d.nnz;
  a.m = d.m;
  a.K = K;
  a.splits = p.splits;
  a.rows_per_split = p.rows_per_split;
  a.nprob = d.nprob;
  char* ws = static_cast<char*>(workspace);
  for (int i = 0; i < d.nprob; ++i) {
    const int src = pair ? 0 : i;  // the pair shares problem 0's plan and output
    const nm_gemv_problem& q = d.prob[src];
    Problem& P = a.prob[i];
    P.mat_data = d.prob[i].mat_data;
    P.mat_index = d.prob[i].mat_index;
    P.out = q.out;
    P.resid = q.residual;
    P.head_w = q.head_norm;
    P.head_stride = q.head_stride;
    P.elem_stride = q.elem_stride;
    P.pos_stride = q.pos_stride;
    P.rope = q.rope;
    P.h = hs[src];
    P.tiles = p.tiles[src];
    P.block_begin = p.block_begin[src];
    P.tickets = reinterpret_cast<uint32_t*>(ws) + p.ticket_off[src];
    P.partial = reinterpret_cast<float*>(ws + p.partial_off[src] +
                                         (size_t)i * (pair ? (size_t)p.splits * (size_t)hs[0] * 4 : 0));
  }
  a.carry_out = d.carry_out;
  a.carry_in = d.carry_in;
  a.vec_out = d.vec_out;
  a.carry_splits = d.carry_splits;
  a.ssq_slots = carry_in ? reinterpret_cast<float*>(ws + p.ssq_off) : nullptr;
  a.carry_acc = d.carry_accumulate;
  a.zero_buf = d.zero_buf;
  a.zero_len = d.zero_len;
  a.silu_in = d.silu_in;
  a.silu_ssq_n = d.silu_ssq_n;
  a.silu_k = d.silu_k;
  a.silu_eps = d.silu_eps;
  const int variant = silu_in    ? kVarSilu
                      : carry_in ? (d.carry_splits == 1 ? kVarCarry1 : (d.carry_splits <= 8 ? kVarCarry8 : kVarCarry16))
                                 : (d.norm_weight ? kVarNorm : kVarPlain);
  const KernelFn fn = kernel_table(d.dtype, pair)[p.cfg].fn[gather_slot(p.rows_per_split)][variant];
  if (!fn) return NM_ERR_BAD_EPILOGUE;
  hipLaunchKernelGGL(fn, dim3(p.blocks), dim3(kBlock), 0, static_cast<hipStream_t>(stream), a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NM_OK : (int)e;
}

nm_gemv_launch_desc plain_desc(int dtype, int kind, const void* vec, int vec_stride, int w, int nnz, int m,
                               int cfg, int splits) {
  nm_gemv_launch_desc d;
  memset(&d, 0, sizeof(d));
  d.dtype = dtype;
  d.kind = kind;
  d.vec = vec;
  d.vec_stride = vec_stride;
  d.w = w;
  d.nnz = nnz;
  d.m = m;
  d.config_id = cfg;
  d.splits = splits;
  return d;
}

int launch_one(int dtype, const void* vec, int vec_stride, const void* mat_data, const uint8_t* mat_index,
               void* out, void* workspace, size_t workspace_bytes, int h, int w, int nnz, int m, int cfg,
               int splits, void* stream) {
  nm_gemv_launch_desc d = plain_desc(dtype, NM_KIND_GROUPED, vec, vec_stride, w, nnz, m, cfg, splits);
  d.nprob = 1;
  d.prob[0].mat_data = mat_data;
  d.prob[0].mat_index = mat_index;
  d.prob[0].out = out;
  d.prob[0].h = h;
  return launch(d, workspace, workspace_bytes, stream, nullptr);
}

// Batch rows per SpMM launch (2, 4 or 8 instantiated; a slot of the table).
inline int spmm_nb_slot(int batch) { return batch <= 2 ? 0 : (batch <= 4 ? 1 : 2); }

const SpmmRow* spmm_table(int dtype) {
  switch (dtype) {
    case NM_DTYPE_F16: return kSpmmKernelsF16;
    case NM_DTYPE_BF16: return kSpmmKernelsBF16;
    default: return kSpmmKernelsF32;
  }
}

// SpMM plan: the GEMV plan of the same configuration (so rows are bitwise the
// GEMV's), with at most kMaxRowsSpmm columns per split and batch-wide partials.
int make_spmm_plan(int batch, int h, int w, int nnz, int m, int cfg, int splits, Plan* p) {
  if (batch < 1 || batch > kMaxBatch) return NM_ERR_BAD_SHAPE;
  if (cfg < 0) {
    const int rc = validate_shape(h, w, nnz, m);
    if (rc != NM_OK) return rc;
    // 256-row tiles past 4096 outputs, as the GEMV, except for short columns
    // at batch > 2 below 8192 outputs; 8-row chunks per lane at batch <= 2, 4
    // above (the FMA work per loaded word grows with the batch). From sweeps
    // at the Llama-3.1-8B and Qwen3-14B shapes.
    const bool wide = h >= 8192 || (h > 4096 && (w >= 6144 || batch <= 2));
    const bool u8 = batch <= 2;
    cfg = (wide ? 2 : 0) + (u8 ? 1 : 0);  // th16_u4, th16_u8, th32_u4, th32_u8
  }
  if (cfg >= kNumSpmmConfigs) return NM_ERR_BAD_CONFIG;
  return make_plan(1, &h, w, nnz, m, 1, cfg, splits, p, kMaxRowsSpmm, batch);
}

int launch_spmm(int dtype, const void* x, long long x_row_stride, int batch, const void* mat_data,
                const uint8_t* mat_index, void* out, long long out_row_stride, void* workspace,
                size_t workspace_bytes, int h, int w, int nnz, int m, int cfg, int splits, void* stream) {
  if (dtype < NM_DTYPE_F16 || dtype > NM_DTYPE_F32) return NM_ERR_BAD_CONFIG;
  Plan p;
  const int rc = make_spmm_plan(batch, h, w, nnz, m, cfg, splits, &p);
  if (rc != NM_OK) return rc;
  if (!x || !mat_data || !mat_index || !out || !workspace) return NM_ERR_NULL_POINTER;
  const long long K = (long long)(w / nnz) * (long long)m;
  if (batch > 1 && (x_row_stride < K || out_row_stride < h)) return NM_ERR_BAD_SHAPE;
  if (((uintptr_t)mat_data & 15u) != 0 || ((uintptr_t)out & 15u) != 0) return NM_ERR_MISALIGNED;
  if (((uintptr_t)workspace & 255u) != 0) return NM_ERR_MISALIGNED;
  if (workspace_bytes < p.workspace) return NM_ERR_WORKSPACE;
  SpmmArgs a;
  memset(&a, 0, sizeof(a));
  a.x = x;
  a.x_row_stride = x_row_stride;
  a.mat_data = mat_data;
  a.mat_index = mat_index;
  a.out = out;
  a.out_row_stride = out_row_stride;
  a.tickets = reinterpret_cast<uint32_t*>(workspace) + p.ticket_off[0];
  a.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + p.partial_off[0]);
  a.batch = batch;
  a.h = h;
  a.tiles = p.tiles[0];
  a.w = w;
  a.nnz = nnz;
  a.m = m;
  a.K = (int)K;
  a.splits = p.splits;
  a.rows_per_split = p.rows_per_split;
  const int gslot = gather_slot(p.rows_per_split);  // <= 2: rows_per_split <= kMaxRowsSpmm
  const SpmmFn fn = spmm_table(dtype)[p.cfg].fn[spmm_nb_slot(batch)][gslot];
  hipLaunchKernelGGL(fn, dim3(p.blocks), dim3(kBlock), 0, static_cast<hipStream_t>(stream), a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NM_OK : (int)e;
}

}  // namespace
}  // namespace nm_hip

// Scratch of nm_gemv_launch_static: arrival counters (the first
// NM_TICKET_BYTES), then split-K partials, in static device memory. Each GPU
// the library runs on holds its own copy until the process ends. In host code
// `scratch` names a host-side stand-in, not device memory: host code uses only
// the per-device address that hipGetSymbolAddress returns for it.
static __device__ __align__(256) unsigned char scratch[NM_STATIC_SCRATCH_BYTES];

namespace nm_hip {
namespace {

// Zero n 32-bit words (the scratch's counters, once per device before its
// first use; a kernel rather than a memset node, so it is also safe to record).
__global__ void clear_words(uint32_t* p, int n) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) p[i] = 0u;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];  // per-device address of `scratch`, set once

// The address of this GPU's scratch (the stream's device, or the current
// device for the null stream), looked up on the first call for that device,
// whose counters are then cleared on `stream`.
int static_scratch(void* stream, void** out) {
  int dev = 0;
  hipError_t e = stream ? hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return NM_ERR_BAD_CONFIG;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    int cur = 0;
    if ((e = hipGetDevice(&cur)) != hipSuccess) return (int)e;
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return (int)e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess && p && ((uintptr_t)p & 255u) == 0) {
      constexpr int kWords = NM_TICKET_BYTES / 4;
      hipLaunchKernelGGL(clear_words, dim3((kWords + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                         static_cast<uint32_t*>(p), kWords);
      e = hipGetLastError();
    }
    if (cur != dev) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess) e = e2;
    }
    if (e != hipSuccess) return (int)e;
    if (!p || ((uintptr_t)p & 255u) != 0) return NM_ERR_MISALIGNED;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return NM_OK;
}

}  // namespace
}  // namespace nm_hip

using namespace nm_hip;

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

size_t nm_gemv_workspace_bytes(int h, int w, int nnz, int m) {
  Plan p;
  return make_plan(1, &h, w, nnz, m, 1, -1, 0, &p) == NM_OK ? p.workspace : 0;
}

size_t nm_gemv_workspace_bytes_ex(int h, int w, int nnz, int m, int config_id, int splits) {
  Plan p;
  return make_plan(1, &h, w, nnz, m, 1, config_id, splits, &p) == NM_OK ? p.workspace : 0;
}

int nm_gemv_f16(const void* vec, int vec_stride, const void* mat_data, const uint8_t* mat_index,
                void* out, void* workspace, size_t workspace_bytes, int h, int w, int nnz, int m,
                void* stream) {
  return launch_one(NM_DTYPE_F16, vec, vec_stride, mat_data, mat_index, out, workspace, workspace_bytes, h,
                    w, nnz, m, -1, 0, stream);
}

int nm_gemv_bf16(const void* vec, int vec_stride, const void* mat_data, const uint8_t* mat_index,
                 void* out, void* workspace, size_t workspace_bytes, int h, int w, int nnz, int m,
                 void* stream) {
  return launch_one(NM_DTYPE_BF16, vec, vec_stride, mat_data, mat_index, out, workspace, workspace_bytes, h,
                    w, nnz, m, -1, 0, stream);
}

int nm_gemv_f32(const void* vec, int vec_stride, const void* mat_data, const uint8_t* mat_index,
                void* out, void* workspace, size_t workspace_bytes, int h, int w, int nnz, int m,
                void* stream) {
  return launch_one(NM_DTYPE_F32, vec, vec_stride, mat_data, mat_index, out, workspace, workspace_bytes, h,
                    w, nnz, m, -1, 0, stream);
}

int nm_gemv_ex(int dtype, const void* vec, int vec_stride, const void* mat_data,
               const uint8_t* mat_index, void* out, void* workspace, size_t workspace_bytes,
               int h, int w, int nnz, int m, int config_id, int splits, void* stream) {
  return launch_one(dtype, vec, vec_stride, mat_data, mat_index, out, workspace, workspace_bytes, h, w, nnz,
                    m, config_id, splits, stream);
}

size_t nm_gemv_grouped_workspace_bytes(int nprob, const int* hs, int w, int nnz, int m, int config_id,
                                       int splits) {
  Plan p;
  if (!hs) return 0;
  return make_plan(nprob, hs, w, nnz, m, 1, config_id, splits, &p) == NM_OK ? p.workspace : 0;
}

int nm_gemv_grouped(int dtype, const void* vec, int vec_stride, int nprob, const void* const* mat_data,
                    const uint8_t* const* mat_index, void* const* out, const int* hs, void* workspace,
                    size_t workspace_bytes, int w, int nnz, int m, int config_id, int splits, void* stream) {
  if (!mat_data || !mat_index || !out || !hs) return NM_ERR_NULL_POINTER;
  if (nprob < 1 || nprob > kMaxProblems) return NM_ERR_BAD_SHAPE;
  nm_gemv_launch_desc d = plain_desc(dtype, NM_KIND_GROUPED, vec, vec_stride, w, nnz, m, config_id, splits);
  d.nprob = nprob;
  for (int i = 0; i < nprob; ++i) {
    d.prob[i].mat_data = mat_data[i];
    d.prob[i].mat_index = mat_index[i];
    d.prob[i].out = out[i];
    d.prob[i].h = hs[i];
  }
  return launch(d, workspace, workspace_bytes, stream, nullptr);
}

size_t nm_gemv_gate_up_workspace_bytes(int h, int w, int nnz, int m, int config_id, int splits) {
  Plan p;
  return make_plan(1, &h, w, nnz, m, 2, config_id, splits, &p) == NM_OK ? p.workspace : 0;
}

int nm_gemv_gate_up_silu(int dtype, const void* vec, int vec_stride, const void* gate_data,
                         const uint8_t* gate_index, const void* up_data, const uint8_t* up_index, void* out,
                         void* workspace, size_t workspace_bytes, int h, int w, int nnz, int m,
                         int config_id, int splits, void* stream) {
  nm_gemv_launch_desc d = plain_desc(dtype, NM_KIND_GATE_UP, vec, vec_stride, w, nnz, m, config_id, splits);
  d.nprob = 2;
  d.prob[0].mat_data = gate_data;
  d.prob[0].mat_index = gate_index;
  d.prob[0].out = out;
  d.prob[0].h = h;
  d.prob[1].mat_data = up_data;
  d.prob[1].mat_index = up_index;
  d.prob[1].h = h;
  return launch(d, workspace, workspace_bytes, stream, nullptr);
}

size_t nm_gemv_launch_workspace_bytes(const nm_gemv_launch_desc* desc) {
  if (!desc) return 0;
  size_t need = 0;
  return launch(*desc, nullptr, 0, nullptr, &need) == NM_OK ? need : 0;
}

int nm_gemv_launch_plan(const nm_gemv_launch_desc* desc, int* out_config_id, int* out_splits, int* out_blocks,
                        int* out_rows_per_split, int* out_chunk_rows) {
  if (!desc) return NM_ERR_NULL_POINTER;
  const bool pair = desc->kind == NM_KIND_GATE_UP;
  if (desc->kind != NM_KIND_GROUPED && !pair) return NM_ERR_BAD_CONFIG;
  const int nprob = pair ? 1 : desc->nprob;
  if (pair ? desc->nprob != 2 : (nprob < 1 || nprob > kMaxProblems)) return NM_ERR_BAD_SHAPE;
  int hs[kMaxProblems];
  for (int i = 0; i < nprob; ++i) hs[i] = desc->prob[i].h;
  Plan p;
  if (desc->nnz <= 0) return NM_ERR_BAD_SHAPE;
  const int rc = plan_desc(*desc, nprob, hs, pair ? 2 : 1, &p);
  if (rc != NM_OK) return rc;
  const Config& c = pair ? kDualConfigs[p.cfg] : kConfigs[p.cfg];
  if (out_config_id) *out_config_id = p.cfg;
  if (out_splits) *out_splits = p.splits;
  if (out_blocks) *out_blocks = p.blocks;
  if (out_rows_per_split) *out_rows_per_split = p.rows_per_split;
  if (out_chunk_rows) *out_chunk_rows = (kBlock / c.th) * c.u;
  return NM_OK;
}

int nm_gemv_launch(const nm_gemv_launch_desc* desc, void* workspace, size_t workspace_bytes, void* stream) {
  if (!desc) return NM_ERR_NULL_POINTER;
  return launch(*desc, workspace, workspace_bytes, stream, nullptr);
}

int nm_gemv_launch_static(const nm_gemv_launch_desc* desc, void* stream) {
  if (!desc) return NM_ERR_NULL_POINTER;
  size_t need = 0;
  int rc = launch(*desc, nullptr, 0, nullptr, &need);  // plan only
  if (rc != NM_OK) return rc;
  if (need > (size_t)NM_STATIC_SCRATCH_BYTES) return NM_ERR_STATIC_SCRATCH;
  // Every argument check before the first HIP call (a 256-byte aligned stand-in
  // for the scratch address, never dereferenced).
  rc = launch(*desc, reinterpret_cast<void*>((uintptr_t)256), NM_STATIC_SCRATCH_BYTES, stream, nullptr, true);
  if (rc != NM_OK) return rc;
  void* ptr = nullptr;
  rc = static_scratch(stream, &ptr);
  if (rc != NM_OK) return rc;
  return launch(*desc, ptr, NM_STATIC_SCRATCH_BYTES, stream, nullptr);
}

size_t nm_spmm_workspace_bytes(int batch, int h, int w, int nnz, int m, int config_id, int splits) {
  Plan p;
  return make_spmm_plan(batch, h, w, nnz, m, config_id, splits, &p) == NM_OK ? p.workspace : 0;
}

int nm_spmm(int dtype, const void* x, long long x_row_stride, int batch, const void* mat_data,
            const uint8_t* mat_index, void* out, long long out_row_stride, void* workspace, size_t workspace_bytes,
            int h, int w, int nnz, int m, int config_id, int splits, void* stream) {
  return launch_spmm(dtype, x, x_row_stride, batch, mat_data, mat_index, out, out_row_stride, workspace,
                     workspace_bytes, h, w, nnz, m, config_id, splits, stream);
}

int nm_spmm_plan(int batch, int h, int w, int nnz, int m, int config_id, int splits, int* out_config_id,
                 int* out_splits, int* out_blocks, int* out_rows_per_block) {
  Plan p;
  const int rc = make_spmm_plan(batch, h, w, nnz, m, config_id, splits, &p);
  if (rc != NM_OK) return rc;
  if (out_config_id) *out_config_id = p.cfg;
  if (out_splits) *out_splits = p.splits;
  if (out_blocks) *out_blocks = p.blocks;
  if (out_rows_per_block) *out_rows_per_block = p.rows_per_split;
  return NM_OK;
}

int nm_num_configs(void) { return kNumConfigs; }

int nm_num_gate_up_configs(void) { return kNumDualConfigs; }

int nm_config_describe(int config_id, char* buf, int buf_len) {
  if (!buf || buf_len <= 0) return NM_ERR_BAD_CONFIG;
  if (config_id >= 0 && config_id < kNumConfigs) {
    const Config& c = kConfigs[config_id];
    snprintf(buf, (size_t)buf_len, "th%d_u%d%s", c.th, c.u, c.nt ? "" : "_cached");
    return NM_OK;
  }
  const int d = config_id - kNumConfigs;
  if (d >= 0 && d < kNumDualConfigs) {
    const Config& c = kDualConfigs[d];
    snprintf(buf, (size_t)buf_len, "pair_th%d_u%d", c.th, c.u);
    return NM_OK;
  }
  return NM_ERR_BAD_CONFIG;
}

int nm_gemv_plan(int h, int w, int nnz, int m, int config_id, int splits, int* out_config_id,
                 int* out_splits, int* out_blocks, int* out_rows_per_block) {
  Plan p;
  int rc = make_plan(1, &h, w, nnz, m, 1, config_id, splits, &p);
  if (rc != NM_OK) return rc;
  if (out_config_id) *out_config_id = p.cfg;
  if (out_splits) *out_splits = p.splits;
  if (out_blocks) *out_blocks = p.blocks;
  if (out_rows_per_block) *out_rows_per_block = p.rows_per_split;
  return NM_OK;
}

const char* nm_strerror(int code) {
  switch (code) {
    case NM_OK: return "success";
    case NM_ERR_NULL_POINTER: return "null device pointer";
    case NM_ERR_BAD_SHAPE: return "shape out of range (h, w, nnz, m, vec_stride, problem count)";
    case NM_ERR_H_NOT_MULTIPLE_128: return "h must be divisible by 128";
    case NM_ERR_W_NOT_MULTIPLE_NNZ: return "w must be divisible by nnz";
    case NM_ERR_MISALIGNED: return "mat_data/out must be 16-byte aligned, workspace 256-byte aligned";
    case NM_ERR_WORKSPACE: return "workspace missing or smaller than the *_workspace_bytes() value";
    case NM_ERR_BAD_CONFIG: return "unknown dtype, launch kind, config id or split count";
    case NM_ERR_STATIC_SCRATCH:
      return "the launch needs more workspace than the static scratch holds (NM_STATIC_SCRATCH_BYTES); use "
             "nm_gemv_launch with a workspace";
    case NM_ERR_BAD_EPILOGUE:
      return "input-norm / residual / head-layout arguments rejected (contiguous 16-byte aligned vec for the "
             "norm; head_dim a multiple of 64 dividing h and the tile; pos and rope table when used)";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "unknown status code";
}

int nm_abi_version(void) { return kAbiVersion; }

int nm_stream_capture_id(void* stream, unsigned long long* out_id) {
  if (!out_id) return NM_ERR_NULL_POINTER;
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  const hipError_t err = hipStreamGetCaptureInfo(static_cast<hipStream_t>(stream), &status, &id);
  if (err != hipSuccess) return (int)err;
  *out_id = status == hipStreamCaptureStatusActive ? id : 0ull;
  return NM_OK;
}

}  // extern "C"
