// nm_gemv.hip — shared-mask N:M sparse GEMV for MI355X (gfx950, CDNA4).
//
// out[r] = RNE_T( sum_{c<w} f32(mat_data[c, r]) * f32(vec[(c/nnz)*m + mat_index[c]]) )
//
// Semantics follow the reference kernels (triton_spmv.py:56-115 and
// triton_spmv.py:149-214): the same packed layout, fp32 fused multiply-add
// accumulation (triton_spmv.py:24-35 is an fma.rn.f32), and an fp32 -> T
// round-to-nearest-even cast of the result (triton_spmv.py:318). The work
// decomposition is this file's own:
//
//  * A workgroup (256 lanes = 4 wave64) owns an output tile of HT = 8*TH
//    consecutive rows r and a contiguous range of compressed columns c
//    (a "split" of w). Lane (tk, th) streams 16 B of every mat_data row it
//    owns (8 fp16/bf16 outputs; 2 x 16 B for fp32), so one wave reads whole
//    128 B lines of each row with dwordx4 non-temporal loads.
//  * The activations a split needs, vec[(c/nnz)*m + mat_index[c]], are
//    gathered once per workgroup into LDS as fp32. Because the mask is shared
//    by all rows, every lane reading row c reads the same LDS word (a
//    broadcast), four rows per ds_read_b128.
//  * Partial sums of the TK lane-rows are reduced through LDS in a fixed
//    order. With more than one split, each workgroup writes its fp32 partial
//    tile to the workspace; the last workgroup to arrive at a tile (an
//    agent-scope arrival counter) adds the partials in split order, rounds to
//    T and writes the output, then re-arms the counter. One launch replaces
//    the reference's zero-fill + atomics + cast kernels and is deterministic.
//
// The C ABI at the bottom is declared in include/nmsparse_hip.h.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/nmsparse_hip.h"

namespace {

constexpr int kBlock = 256;        // lanes per workgroup
constexpr int kVec = 8;            // output rows per lane
constexpr int kMaxRows = 2048;     // compressed columns per split (LDS gather bound)
constexpr int kMaxTickets = NM_TICKET_BYTES / 4;
constexpr int kAbiVersion = 1;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------------------
// Element types. Raw rows are kept as 16 B words until the FMA so that the
// loads of a whole chunk can be in flight at once.
// ---------------------------------------------------------------------------
template <int DT>
struct Elem;

template <>
struct Elem<NM_DTYPE_F16> {
  static constexpr int kWords = 1;  // 16 B words per 8 elements
  typedef uint16_t scalar;
  __device__ static inline float to_f32(scalar v) {
    return (float)__builtin_bit_cast(_Float16, v);
  }
  __device__ static inline scalar from_f32(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
  // Whole-vector bitcast: a bitcast of a single vector element read through
  // an array reference loses the element index in this compiler.
  __device__ static inline void unpack(const u32x4 (&raw)[1], float (&v)[8]) {
    const f16x8 p = __builtin_bit_cast(f16x8, raw[0]);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)p[i];
  }
};

template <>
struct Elem<NM_DTYPE_BF16> {
  static constexpr int kWords = 1;
  typedef uint16_t scalar;
  __device__ static inline float to_f32(scalar v) {
    return __uint_as_float(((uint32_t)v) << 16);
  }
  // Round to nearest, ties to even, on the bit pattern; NaN -> quiet NaN.
  __device__ static inline scalar from_f32(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (scalar)0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (scalar)(u >> 16);
  }
  __device__ static inline void unpack(const u32x4 (&raw)[1], float (&v)[8]) {
    const u32x4 r = raw[0];
    const uint32_t d[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(d[i] << 16);
      v[2 * i + 1] = __uint_as_float(d[i] & 0xffff0000u);
    }
  }
};

template <>
struct Elem<NM_DTYPE_F32> {
  static constexpr int kWords = 2;
  typedef float scalar;
  __device__ static inline float to_f32(scalar v) { return v; }
  __device__ static inline scalar from_f32(float f) { return f; }
  __device__ static inline void unpack(const u32x4 (&raw)[2], float (&v)[8]) {
    const u32x4 lo = raw[0];
    const u32x4 hi = raw[1];
    const uint32_t d[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(d[i]);
  }
};

template <bool NT>
__device__ inline u32x4 load16(const u32x4* p) {
  if constexpr (NT) {
    return __builtin_nontemporal_load(p);
  } else {
    return *p;
  }
}

// ---------------------------------------------------------------------------
// Kernel
// ---------------------------------------------------------------------------
struct Args {
  const void* vec;
  const void* mat_data;
  const uint8_t* mat_index;
  void* out;
  float* partial;      // [splits, h] fp32, unused when splits == 1
  uint32_t* tickets;   // [tiles] arrival counters, zero between launches
  long long vec_stride;
  int h;
  int w;
  int nnz;
  int m;
  int K;
  int tiles;
  int splits;
  int rows_per_split;  // multiple of the chunk height, <= kMaxRows
};

template <int DT, int TH, int U, int G, bool NT>
__global__ __launch_bounds__(kBlock) void nm_gemv_kernel(Args a) {
  using E = Elem<DT>;
  typedef typename E::scalar T;
  constexpr int W = E::kWords;
  constexpr int TK = kBlock / TH;   // lane-rows per workgroup
  constexpr int HT = TH * kVec;     // output rows per tile
  constexpr int CH = TK * U;        // compressed columns per chunk
  constexpr int XR = G * kBlock;    // compressed columns per split (max)
  static_assert(kBlock % TH == 0, "TH must divide the block");
  static_assert(U % 4 == 0, "U must be a multiple of 4 (ds_read_b128)");
  static_assert(XR % CH == 0, "chunk must divide the split");

  __shared__ __attribute__((aligned(16))) float xs[XR];
  __shared__ __attribute__((aligned(16))) float red[TK * HT];
  __shared__ int is_last;

  const int tid = threadIdx.x;
  const int th = tid % TH;
  const int tk = tid / TH;
  const int tile = blockIdx.x % a.tiles;
  const int split = blockIdx.x / a.tiles;
  const int c0 = split * a.rows_per_split;
  const int cw = min(a.rows_per_split, a.w - c0);  // 1 <= cw <= XR by construction
  const int nch = (cw + CH - 1) / CH;
  const int col = tile * HT + th * kVec;
  // Lanes past the last output row read a valid column instead (their sums
  // are never stored), so no weight load needs a branch.
  const int col_ld = min(col, a.h - kVec);

  const T* __restrict__ md = static_cast<const T*>(a.mat_data);
  const T* __restrict__ vx = static_cast<const T*>(a.vec);
  const uint8_t* __restrict__ mi = a.mat_index;
  const T* __restrict__ md_tile = md + (size_t)c0 * (size_t)a.h + (size_t)col_ld;

  // All loads below are unconditional (addresses clamped into range) so that
  // the compiler keeps them in flight together; out-of-range values are
  // zeroed with selects after they arrive.

  // 1. In-group positions of this split's compressed columns. mat_index is
  //    [w/nnz, nnz] contiguous, so column c's position is mi[c].
  int gidx[G];
#pragma unroll
  for (int j = 0; j < G; ++j) gidx[j] = (int)mi[c0 + min(tid + j * kBlock, cw - 1)];

  // 2. The first chunk of weights goes in flight before the activation loads.
  auto load_chunk = [&](u32x4 (&dst)[U][W], int k) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = min(k * CH + tk * U + u, cw - 1);
      const u32x4* p = reinterpret_cast<const u32x4*>(md_tile + (size_t)r * (size_t)a.h);
#pragma unroll
      for (int q = 0; q < W; ++q) dst[u][q] = load16<NT>(p + q);
    }
  };
  u32x4 bufA[U][W];
  u32x4 bufB[U][W];
  load_chunk(bufA, 0);

  // 3. Gather the activations: vec[(c/nnz)*m + position], fp32 in LDS. Rows
  //    past the split and positions outside vec read as zero.
  T graw[G];
  bool gok[G];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const int t = tid + j * kBlock;
    const int c = c0 + min(t, cw - 1);
    const int pos = (c / a.nnz) * a.m + gidx[j];
    gok[j] = (t < cw) && (pos < a.K);
    graw[j] = vx[(long long)(gok[j] ? pos : 0) * a.vec_stride];
  }
#pragma unroll
  for (int j = 0; j < G; ++j) xs[tid + j * kBlock] = gok[j] ? E::to_f32(graw[j]) : 0.0f;
  __syncthreads();

  float acc[kVec];
#pragma unroll
  for (int e = 0; e < kVec; ++e) acc[e] = 0.0f;

  // FMA one chunk; rows past the split contribute exactly nothing.
  auto fma_chunk = [&](const u32x4 (&src)[U][W], int k) {
    const int r0 = k * CH + tk * U;
#pragma unroll
    for (int u4 = 0; u4 < U / 4; ++u4) {
      const float4 xv = *reinterpret_cast<const float4*>(&xs[r0 + 4 * u4]);
      const float xq[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bool ok = (r0 + 4 * u4 + s) < cw;
        u32x4 rw[W];
#pragma unroll
        for (int q = 0; q < W; ++q)
          rw[q] = ok ? src[4 * u4 + s][q] : u32x4{0u, 0u, 0u, 0u};
        float v[kVec];
        E::unpack(rw, v);
#pragma unroll
        for (int e = 0; e < kVec; ++e) acc[e] = __builtin_fmaf(v[e], xq[s], acc[e]);
      }
    }
  };

  // 4. Stream the split two chunks at a time: chunk k+1 is in flight while
  //    chunk k is consumed. Loads inside the loop are unconditional.
  int k = 0;
  for (; k + 2 < nch; k += 2) {
    load_chunk(bufB, k + 1);
    fma_chunk(bufA, k);
    load_chunk(bufA, k + 2);
    fma_chunk(bufB, k + 1);
  }
  if (k + 1 < nch) {
    load_chunk(bufB, k + 1);
    fma_chunk(bufA, k);
    fma_chunk(bufB, k + 1);
  } else {
    fma_chunk(bufA, k);
  }

  // 5. Reduce the TK lane-rows of the tile through LDS (fixed order).
  {
    float4* rp = reinterpret_cast<float4*>(&red[tk * HT + th * kVec]);
    rp[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    rp[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
  __syncthreads();

  T* __restrict__ out = static_cast<T*>(a.out);
  constexpr int kOutPerLane = (HT + kBlock - 1) / kBlock;
  float tsum[kOutPerLane];
#pragma unroll
  for (int j = 0; j < kOutPerLane; ++j) {
    const int o = tid + j * kBlock;
    float s = 0.0f;
    if (o < HT) {
#pragma unroll
      for (int q = 0; q < TK; ++q) s += red[q * HT + o];
    }
    tsum[j] = s;
  }

  if (a.splits == 1) {
#pragma unroll
    for (int j = 0; j < kOutPerLane; ++j) {
      const int o = tid + j * kBlock;
      const int r = tile * HT + o;
      if (o < HT && r < a.h) out[r] = E::from_f32(tsum[j]);
    }
    return;
  }

  // 6. Split-K: publish the partial tile, count arrivals, last one reduces.
  //    The handoff uses agent-scope atomics only, never an agent-scope fence:
  //    on gfx950 such a fence writes back and invalidates the whole L2 of the
  //    workgroup's XCD (buffer_wbl2 / buffer_inv), which costs more than the
  //    GEMV itself. Each partial is published with a returning atomic swap:
  //    its result comes back only after the swap has been performed at the
  //    device coherence point, and each lane waits for all of its results
  //    (vmcnt(0)) before the barrier. Lane 0 then counts the arrival; the
  //    last arrival reads every partial with agent-scope atomic loads (sc1,
  //    coherent across XCDs) in split order, so the sum is deterministic.
  float sink = 0.0f;
#pragma unroll
  for (int j = 0; j < kOutPerLane; ++j) {
    const int o = tid + j * kBlock;
    const int r = tile * HT + o;
    if (o < HT && r < a.h)
      sink += __hip_atomic_exchange(a.partial + (size_t)split * (size_t)a.h + (size_t)r, tsum[j],
                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // Consume the swap results (a.splits is never negative) so the compiler
  // keeps the returning form of the instruction.
  if (a.splits < 0) out[tid] = E::from_f32(sink);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&a.tickets[tile], 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    is_last = (prev == (uint32_t)(a.splits - 1)) ? 1 : 0;
  }
  __syncthreads();
  if (!is_last) return;

#pragma unroll
  for (int j = 0; j < kOutPerLane; ++j) {
    const int o = tid + j * kBlock;
    const int r = tile * HT + o;
    if (o < HT && r < a.h) {
      float* p = a.partial + r;
      float s = 0.0f;
      int sp = 0;
      for (; sp + 8 <= a.splits; sp += 8) {
        float t[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
          t[q] = __hip_atomic_load(p + (size_t)(sp + q) * (size_t)a.h, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int q = 0; q < 8; ++q) s += t[q];
      }
      for (; sp < a.splits; ++sp)
        s += __hip_atomic_load(p + (size_t)sp * (size_t)a.h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      out[r] = E::from_f32(s);
    }
  }
  if (tid == 0) {
    __hip_atomic_store(&a.tickets[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------
// Configuration table (static; no runtime autotuning).
// ---------------------------------------------------------------------------
typedef void (*KernelFn)(Args);

struct Config {
  int th;       // lanes along the output rows (tile = 8*th rows)
  int u;        // rows per lane per chunk
  bool nt;      // non-temporal weight loads
  KernelFn fn[3][4];  // [dtype][gather width: 256, 512, 1024, 2048 columns per split]
};

#define NM_CFG_G(DT, TH, U, NT)                                               \
  {&nm_gemv_kernel<DT, TH, U, 1, NT>, &nm_gemv_kernel<DT, TH, U, 2, NT>,       \
   &nm_gemv_kernel<DT, TH, U, 4, NT>, &nm_gemv_kernel<DT, TH, U, 8, NT>}
#define NM_CFG(TH, U, NT)                                                     \
  {TH, U, NT,                                                                 \
   {NM_CFG_G(NM_DTYPE_F16, TH, U, NT), NM_CFG_G(NM_DTYPE_BF16, TH, U, NT),   \
    NM_CFG_G(NM_DTYPE_F32, TH, U, NT)}}

const Config kConfigs[] = {
    NM_CFG(16, 4, true),   // 0: tile 128,  chunk 64
    NM_CFG(16, 8, true),   // 1: tile 128,  chunk 128
    NM_CFG(32, 4, true),   // 2: tile 256,  chunk 32
    NM_CFG(32, 8, true),   // 3: tile 256,  chunk 64
    NM_CFG(32, 16, true),  // 4: tile 256,  chunk 128
    NM_CFG(64, 4, true),   // 5: tile 512,  chunk 16
    NM_CFG(64, 8, true),   // 6: tile 512,  chunk 32
    NM_CFG(64, 16, true),  // 7: tile 512,  chunk 64
    NM_CFG(128, 8, true),  // 8: tile 1024, chunk 16
    NM_CFG(256, 8, true),  // 9: tile 2048, chunk 8
    NM_CFG(16, 8, false),  // 10: as 1, cached loads
    NM_CFG(32, 8, false),  // 11: as 3, cached loads
    NM_CFG(64, 8, false),  // 12: as 6, cached loads
};
constexpr int kNumConfigs = sizeof(kConfigs) / sizeof(kConfigs[0]);

inline int gather_slot(int rows) {
  return rows <= kBlock ? 0 : (rows <= 2 * kBlock ? 1 : (rows <= 4 * kBlock ? 2 : 3));
}

struct Plan {
  int cfg;
  int tiles;
  int splits;
  int rows_per_split;
  int blocks;
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

// The library's own choice of configuration for a shape, from rocprof /
// hipGraph sweeps on MI355X at the Llama-3.1-8B decode shapes: 256-row tiles
// for wide outputs, 128-row tiles otherwise.
int auto_config(int h, int w) {
  (void)w;
  return h >= 8192 ? 3 : 1;
}

// Default split count: about 8 splits of the compressed columns per tile. The
// sweeps show the cost of a split-K handoff (one partial publish, one arrival
// atomic on a per-tile counter, one reduction) grows faster with the split
// count than the extra parallelism pays back; 8 splits of 256+ columns keep
// 64-900 workgroups streaming for every decode shape.
constexpr int kDefaultSplits = 8;

int make_plan(int h, int w, int nnz, int m, int cfg, int splits, Plan* p) {
  int rc = validate_shape(h, w, nnz, m);
  if (rc != NM_OK) return rc;
  if (cfg < 0) cfg = auto_config(h, w);
  if (cfg >= kNumConfigs) return NM_ERR_BAD_CONFIG;
  const Config& c = kConfigs[cfg];
  const int HT = c.th * kVec;
  const int CH = (kBlock / c.th) * c.u;
  const int tiles = ceil_div(h, HT);
  if (tiles > kMaxTickets) return NM_ERR_BAD_SHAPE;
  if (splits <= 0) splits = kDefaultSplits;
  if (splits > w) splits = w;
  int rows = ceil_div(ceil_div(w, splits), CH) * CH;
  if (rows > kMaxRows) rows = kMaxRows;
  if (rows < CH) rows = CH;
  splits = ceil_div(w, rows);
  p->cfg = cfg;
  p->tiles = tiles;
  p->splits = splits;
  p->rows_per_split = rows;
  const long long blocks = (long long)tiles * (long long)splits;
  if (blocks > 0x7fffffffLL) return NM_ERR_BAD_SHAPE;
  p->blocks = (int)blocks;
  p->workspace = (size_t)NM_TICKET_BYTES +
                 (splits > 1 ? (size_t)splits * (size_t)h * sizeof(float) : 0);
  return NM_OK;
}

int launch(int dtype, const void* vec, int vec_stride, const void* mat_data,
           const uint8_t* mat_index, void* out, void* workspace, size_t workspace_bytes,
           int h, int w, int nnz, int m, int cfg, int splits, void* stream) {
  if (dtype < NM_DTYPE_F16 || dtype > NM_DTYPE_F32) return NM_ERR_BAD_CONFIG;
  if (!vec || !mat_data || !mat_index || !out || !workspace) return NM_ERR_NULL_POINTER;
  if (vec_stride < 1) return NM_ERR_BAD_SHAPE;
  Plan p;
  int rc = make_plan(h, w, nnz, m, cfg, splits, &p);
  if (rc != NM_OK) return rc;
  if (((uintptr_t)mat_data & 15u) != 0 || ((uintptr_t)out & 15u) != 0) return NM_ERR_MISALIGNED;
  if (((uintptr_t)workspace & 255u) != 0) return NM_ERR_MISALIGNED;
  if (workspace_bytes < p.workspace) return NM_ERR_WORKSPACE;

  Args a;
  a.vec = vec;
  a.mat_data = mat_data;
  a.mat_index = mat_index;
  a.out = out;
  a.tickets = static_cast<uint32_t*>(workspace);
  a.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + NM_TICKET_BYTES);
  a.vec_stride = vec_stride;
  a.h = h;
  a.w = w;
  a.nnz = nnz;
  a.m = m;
  a.K = (w / nnz) * m;
  a.tiles = p.tiles;
  a.splits = p.splits;
  a.rows_per_split = p.rows_per_split;

  hipLaunchKernelGGL(kConfigs[p.cfg].fn[dtype][gather_slot(p.rows_per_split)], dim3(p.blocks), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NM_OK : (int)e;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

size_t nm_gemv_workspace_bytes(int h, int w, int nnz, int m) {
  Plan p;
  return make_plan(h, w, nnz, m, -1, 0, &p) == NM_OK ? p.workspace : 0;
}

size_t nm_gemv_workspace_bytes_ex(int h, int w, int nnz, int m, int config_id, int splits) {
  Plan p;
  return make_plan(h, w, nnz, m, config_id, splits, &p) == NM_OK ? p.workspace : 0;
}

int nm_gemv_f16(const void* vec, int vec_stride, const void* mat_data, const uint8_t* mat_index,
                void* out, void* workspace, size_t workspace_bytes, int h, int w, int nnz, int m,
                void* stream) {
  return launch(NM_DTYPE_F16, vec, vec_stride, mat_data, mat_index, out, workspace,
                workspace_bytes, h, w, nnz, m, -1, 0, stream);
}

int nm_gemv_bf16(const void* vec, int vec_stride, const void* mat_data, const uint8_t* mat_index,
                 void* out, void* workspace, size_t workspace_bytes, int h, int w, int nnz, int m,
                 void* stream) {
  return launch(NM_DTYPE_BF16, vec, vec_stride, mat_data, mat_index, out, workspace,
                workspace_bytes, h, w, nnz, m, -1, 0, stream);
}

int nm_gemv_f32(const void* vec, int vec_stride, const void* mat_data, const uint8_t* mat_index,
                void* out, void* workspace, size_t workspace_bytes, int h, int w, int nnz, int m,
                void* stream) {
  return launch(NM_DTYPE_F32, vec, vec_stride, mat_data, mat_index, out, workspace,
                workspace_bytes, h, w, nnz, m, -1, 0, stream);
}

int nm_gemv_ex(int dtype, const void* vec, int vec_stride, const void* mat_data,
               const uint8_t* mat_index, void* out, void* workspace, size_t workspace_bytes,
               int h, int w, int nnz, int m, int config_id, int splits, void* stream) {
  return launch(dtype, vec, vec_stride, mat_data, mat_index, out, workspace, workspace_bytes, h,
                w, nnz, m, config_id, splits, stream);
}

int nm_num_configs(void) { return kNumConfigs; }

int nm_config_describe(int config_id, char* buf, int buf_len) {
  if (config_id < 0 || config_id >= kNumConfigs || !buf || buf_len <= 0) return NM_ERR_BAD_CONFIG;
  const Config& c = kConfigs[config_id];
  snprintf(buf, (size_t)buf_len, "th%d_u%d%s", c.th, c.u, c.nt ? "" : "_cached");
  return NM_OK;
}

int nm_gemv_plan(int h, int w, int nnz, int m, int config_id, int splits, int* out_config_id,
                 int* out_splits, int* out_blocks, int* out_rows_per_block) {
  Plan p;
  int rc = make_plan(h, w, nnz, m, config_id, splits, &p);
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
    case NM_ERR_BAD_SHAPE: return "shape out of range (h, w, nnz, m, vec_stride)";
    case NM_ERR_H_NOT_MULTIPLE_128: return "h must be divisible by 128";
    case NM_ERR_W_NOT_MULTIPLE_NNZ: return "w must be divisible by nnz";
    case NM_ERR_MISALIGNED: return "mat_data/out must be 16-byte aligned, workspace 256-byte aligned";
    case NM_ERR_WORKSPACE: return "workspace missing or smaller than nm_gemv_workspace_bytes()";
    case NM_ERR_BAD_CONFIG: return "unknown dtype, config id or split count";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "unknown status code";
}

int nm_abi_version(void) { return kAbiVersion; }

}  // extern "C"
