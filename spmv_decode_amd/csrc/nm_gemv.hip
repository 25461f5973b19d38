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
constexpr int kAbiVersion = 3;

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
constexpr int kMaxProblems = 4;

// One GEMV of a launch. The problems of one launch share the activation
// vector and K, nnz, m (hence w); their output widths h may differ.
struct Problem {
  const void* mat_data;
  const uint8_t* mat_index;
  void* out;
  float* partial;      // [splits, h] fp32, unused when splits == 1
  uint32_t* tickets;   // [tiles] arrival counters, zero between launches
  const void* resid;   // optional [h] residual added before the rounding
  const void* head_w;  // optional [head_dim] per-head RMSNorm weight
  // Output element of row r: out + (r / head_dim) * head_stride
  //   + (r % head_dim) * elem_stride + pos * pos_stride (heads layout), or
  // out + r when all three are zero.
  long long head_stride;
  long long elem_stride;
  long long pos_stride;
  int h;
  int tiles;
  int block_begin;     // first workgroup of this problem in the grid
  int rope;            // rotate (even, odd) row pairs of each head by pos
};

struct Args {
  const void* vec;
  long long vec_stride;
  const void* norm_w;  // optional [K] RMSNorm weight of the input (folded into the gather)
  const float2* rope;  // [pos_limit, head_dim / 2] (cos, sin) when a problem rotates
  const long long* pos;  // device position for the heads layout / rotation
  float norm_eps;
  float head_eps;
  int head_dim;
  int pos_limit;       // positions >= pos_limit (or < 0) store nothing
  int w;
  int nnz;
  int m;
  int K;
  int splits;
  int rows_per_split;  // multiple of the chunk height, <= kMaxRows
  int nprob;           // NMAT == 1: problems in the grid; NMAT == 2: 2 (gate, up)
  Problem prob[kMaxProblems];
};

__device__ inline float silu(float g) { return g / (1.0f + expf(-g)); }

// NMAT == 1: each workgroup computes one tile/split of one problem (a plain
// GEMV when nprob == 1, several GEMVs sharing x in one grid otherwise).
// NMAT == 2: each workgroup streams the same tile/split of prob[0] (gate) and
// prob[1] (up), both of width prob[0].h, and the output prob[0].out receives
// silu(gate) * up, computed in fp32 and rounded once.
template <int DT, int TH, int U, int G, bool NT, int NMAT>
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
  static_assert(NMAT == 1 || NMAT == 2, "one matrix, or the gate/up pair");

  constexpr int kWaves = kBlock / 64;
  constexpr int kOutPerLane = (HT + kBlock - 1) / kBlock;
  __shared__ __attribute__((aligned(16))) float xs[NMAT][XR];
  __shared__ __attribute__((aligned(16))) float red[NMAT][TK * HT];
  __shared__ float wsum[kOutPerLane * kWaves];  // per-wave sums (input norm, head norms)
  __shared__ int is_last;

  // Problem of this workgroup (uniform; at most kMaxProblems entries).
  int p = 0;
  if (NMAT == 1) {
#pragma unroll
    for (int q = 1; q < kMaxProblems; ++q)
      if (q < a.nprob && (int)blockIdx.x >= a.prob[q].block_begin) p = q;
  }
  const int h = a.prob[p].h;
  const int tiles = a.prob[p].tiles;
  const int local = (int)blockIdx.x - a.prob[p].block_begin;

  const int tid = threadIdx.x;
  const int th = tid % TH;
  const int tk = tid / TH;
  const int tile = local % tiles;
  const int split = local / tiles;
  const int c0 = split * a.rows_per_split;
  const int cw = min(a.rows_per_split, a.w - c0);  // 1 <= cw <= XR by construction
  const int nch = (cw + CH - 1) / CH;
  const int col = tile * HT + th * kVec;
  // Lanes past the last output row read a valid column instead (their sums
  // are never stored), so no weight load needs a branch.
  const int col_ld = min(col, h - kVec);

  const T* __restrict__ vx = static_cast<const T*>(a.vec);
  const T* md_tile[NMAT];
  const uint8_t* mi[NMAT];
#pragma unroll
  for (int q = 0; q < NMAT; ++q) {
    const Problem& P = a.prob[NMAT == 1 ? p : q];
    md_tile[q] = static_cast<const T*>(P.mat_data) + (size_t)c0 * (size_t)h + (size_t)col_ld;
    mi[q] = P.mat_index;
  }

  // All loads below are unconditional (addresses clamped into range) so that
  // the compiler keeps them in flight together; out-of-range values are
  // zeroed with selects after they arrive.

  // 1. In-group positions of this split's compressed columns. mat_index is
  //    [w/nnz, nnz] contiguous, so column c's position is mi[c].
  int gidx[NMAT][G];
#pragma unroll
  for (int q = 0; q < NMAT; ++q)
#pragma unroll
    for (int j = 0; j < G; ++j) gidx[q][j] = (int)mi[q][c0 + min(tid + j * kBlock, cw - 1)];

  // 2. The first chunk of weights goes in flight before the activation loads.
  auto load_chunk = [&](u32x4 (&dst)[NMAT][U][W], int k) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = min(k * CH + tk * U + u, cw - 1);
#pragma unroll
      for (int q = 0; q < NMAT; ++q) {
        const u32x4* ptr = reinterpret_cast<const u32x4*>(md_tile[q] + (size_t)r * (size_t)h);
#pragma unroll
        for (int v = 0; v < W; ++v) dst[q][u][v] = load16<NT>(ptr + v);
      }
    }
  };
  u32x4 bufA[NMAT][U][W];
  u32x4 bufB[NMAT][U][W];
  load_chunk(bufA, 0);

  // 3. Gather the activations: vec[(c/nnz)*m + position], fp32 in LDS. Rows
  //    past the split and positions outside vec read as zero.
  //    With an input RMSNorm, rmsnorm(x) = s * (x * g) with the scalar
  //    s = 1 / sqrt(mean(x^2) + eps): the gather reads x * g and s scales the
  //    finished sums.
  const bool has_norm = a.norm_w != nullptr;
  const T* __restrict__ gx = static_cast<const T*>(has_norm ? a.norm_w : a.vec);
  T graw[NMAT][G];
  T wraw[NMAT][G];
  bool gok[NMAT][G];
#pragma unroll
  for (int q = 0; q < NMAT; ++q)
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int t = tid + j * kBlock;
      const int c = c0 + min(t, cw - 1);
      const int pos = (c / a.nnz) * a.m + gidx[q][j];
      gok[q][j] = (t < cw) && (pos < a.K);
      graw[q][j] = vx[(long long)(gok[q][j] ? pos : 0) * a.vec_stride];
      if (has_norm) wraw[q][j] = gx[gok[q][j] ? pos : 0];
    }
  // Sum of squares of the whole input for s (vec is contiguous and 16-byte
  // aligned with K * sizeof(T) a multiple of 16 when has_norm; the host
  // checks). Every workgroup computes it, in a fixed order.
  float ssq = 0.0f;
  if (has_norm) {
    const u32x4* xw = static_cast<const u32x4*>(a.vec);
    const int nw = (int)(((long long)a.K * (long long)sizeof(T)) / 16);  // 16-byte words of vec
    for (int base = 0; base < nw; base += 4 * kBlock) {
      u32x4 raw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) raw[i] = xw[min(base + i * kBlock + tid, nw - 1)];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = base + i * kBlock + tid < nw;
        float f[8];
        if constexpr (W == 1) {
          const u32x4 one[1] = {raw[i]};
          E::unpack(one, f);
        } else {
          const u32x4 r4 = raw[i];
          const uint32_t d[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) f[e] = __uint_as_float(d[e]);
#pragma unroll
          for (int e = 4; e < 8; ++e) f[e] = 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float fe = ok ? f[e] : 0.0f;
          ssq = __builtin_fmaf(fe, fe, ssq);
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < NMAT; ++q)
#pragma unroll
    for (int j = 0; j < G; ++j) {
      float xv = gok[q][j] ? E::to_f32(graw[q][j]) : 0.0f;
      if (has_norm) xv *= E::to_f32(wraw[q][j]);
      xs[q][tid + j * kBlock] = xv;
    }
  if (has_norm) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ssq += __shfl_xor(ssq, off, 64);
    if ((tid & 63) == 0) wsum[tid >> 6] = ssq;
  }
  __syncthreads();
  float s_in = 1.0f;
  if (has_norm) {
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) t += wsum[i];
    s_in = rsqrtf(t / (float)a.K + a.norm_eps);
  }

  float acc[NMAT][kVec];
#pragma unroll
  for (int q = 0; q < NMAT; ++q)
#pragma unroll
    for (int e = 0; e < kVec; ++e) acc[q][e] = 0.0f;

  // FMA one chunk; rows past the split contribute exactly nothing.
  auto fma_chunk = [&](const u32x4 (&src)[NMAT][U][W], int k) {
    const int r0 = k * CH + tk * U;
#pragma unroll
    for (int q = 0; q < NMAT; ++q) {
#pragma unroll
      for (int u4 = 0; u4 < U / 4; ++u4) {
        const float4 xv = *reinterpret_cast<const float4*>(&xs[q][r0 + 4 * u4]);
        const float xq[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bool ok = (r0 + 4 * u4 + s) < cw;
          u32x4 rw[W];
#pragma unroll
          for (int v = 0; v < W; ++v) rw[v] = ok ? src[q][4 * u4 + s][v] : u32x4{0u, 0u, 0u, 0u};
          float wv[kVec];
          E::unpack(rw, wv);
#pragma unroll
          for (int e = 0; e < kVec; ++e) acc[q][e] = __builtin_fmaf(wv[e], xq[s], acc[q][e]);
        }
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
#pragma unroll
  for (int q = 0; q < NMAT; ++q) {
    float4* rp = reinterpret_cast<float4*>(&red[q][tk * HT + th * kVec]);
    rp[0] = make_float4(acc[q][0], acc[q][1], acc[q][2], acc[q][3]);
    rp[1] = make_float4(acc[q][4], acc[q][5], acc[q][6], acc[q][7]);
  }
  __syncthreads();

  const Problem& P = a.prob[p];
  float tsum[NMAT][kOutPerLane];
#pragma unroll
  for (int q = 0; q < NMAT; ++q)
#pragma unroll
    for (int j = 0; j < kOutPerLane; ++j) {
      const int o = tid + j * kBlock;
      float s = 0.0f;
      if (o < HT) {
#pragma unroll
        for (int t = 0; t < TK; ++t) s += red[q][t * HT + o];
      }
      tsum[q][j] = s;
    }

  uint32_t* tickets = P.tickets;
  if (a.splits > 1) {
    // 6. Split-K: publish the partial tile, count arrivals, last one reduces.
    //    The handoff uses agent-scope atomics only, never an agent-scope
    //    fence: on gfx950 such a fence writes back and invalidates the whole
    //    L2 of the workgroup's XCD (buffer_wbl2 / buffer_inv), which costs
    //    more than the GEMV itself. Each partial is published with a
    //    returning atomic swap: its result comes back only after the swap has
    //    been performed at the device coherence point, and each lane waits
    //    for all of its results (vmcnt(0)) before the barrier. Lane 0 then
    //    counts the arrival; the last arrival reads every partial with
    //    agent-scope atomic loads (sc1, coherent across XCDs) in split order,
    //    so the sum is deterministic.
    float sink = 0.0f;
#pragma unroll
    for (int q = 0; q < NMAT; ++q) {
      float* part = a.prob[NMAT == 1 ? p : q].partial + (size_t)split * (size_t)h;
#pragma unroll
      for (int j = 0; j < kOutPerLane; ++j) {
        const int o = tid + j * kBlock;
        const int r = tile * HT + o;
        if (o < HT && r < h)
          sink += __hip_atomic_exchange(part + r, tsum[q][j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // Consume the swap results (a.splits is never negative) so the compiler
    // keeps the returning form of the instruction.
    if (a.splits < 0) static_cast<T*>(P.out)[tid] = E::from_f32(sink);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(&tickets[tile], 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      is_last = (prev == (uint32_t)(a.splits - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (!is_last) return;
  }

  // 7. Epilogue of the workgroup that owns the finished tile. Its operands
  //    (residual, head-norm weights, position, rotation) are loaded first so
  //    that they are in flight together with the partial sums.
  const int hd = a.head_dim;
  const bool heads = NMAT == 1 && (P.head_w != nullptr || P.rope != 0);
  const bool head_layout = (P.head_stride | P.elem_stride | P.pos_stride) != 0;
  const bool need_pos = P.rope != 0 || P.pos_stride != 0;
  long long pos = 0;
  if (need_pos) pos = *a.pos;
  const bool pos_ok = !need_pos || (pos >= 0 && pos < (long long)a.pos_limit);
  const long long pos_c = pos_ok ? pos : 0;
  const T* __restrict__ resid = static_cast<const T*>(P.resid);
  const T* __restrict__ head_w = static_cast<const T*>(P.head_w);
  float rv[kOutPerLane], hw[kOutPerLane];
  float2 cs[kOutPerLane];
#pragma unroll
  for (int j = 0; j < kOutPerLane; ++j) {
    const int o = tid + j * kBlock;
    const int r = min(tile * HT + min(o, HT - 1), h - 1);  // clamped: loads stay in range
    rv[j] = resid ? E::to_f32(resid[r]) : 0.0f;
    hw[j] = 1.0f;
    cs[j] = make_float2(1.0f, 0.0f);
    if (heads) {
      if (head_w) hw[j] = E::to_f32(head_w[r % hd]);
      if (P.rope) cs[j] = a.rope[pos_c * (long long)(hd / 2) + (r % hd) / 2];
    }
  }
  if (a.splits > 1) {
#pragma unroll
    for (int j = 0; j < kOutPerLane; ++j) {
      const int o = tid + j * kBlock;
      const int r = tile * HT + o;
      if (o < HT && r < h) {
#pragma unroll
        for (int q = 0; q < NMAT; ++q) {
          float* pp = a.prob[NMAT == 1 ? p : q].partial + r;
          float s = 0.0f;
          int sp = 0;
          for (; sp + 8 <= a.splits; sp += 8) {
            float t8[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
              t8[i] = __hip_atomic_load(pp + (size_t)(sp + i) * (size_t)h, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int i = 0; i < 8; ++i) s += t8[i];
          }
          for (; sp < a.splits; ++sp)
            s += __hip_atomic_load(pp + (size_t)sp * (size_t)h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          tsum[q][j] = s;
        }
      }
    }
  }

  float val[kOutPerLane];
#pragma unroll
  for (int j = 0; j < kOutPerLane; ++j) {
    const int o = tid + j * kBlock;
    const bool valid = o < HT && tile * HT + o < h;
    float v;
    if constexpr (NMAT == 1) {
      v = tsum[0][j] * s_in;
    } else {
      v = silu(tsum[0][j] * s_in) * (tsum[1][j] * s_in);
    }
    val[j] = valid ? v : 0.0f;
  }

  if (heads) {
    // Per-head RMSNorm over head_dim consecutive rows (head_dim is a multiple
    // of 64 dividing the tile, so a head is whole waves of this workgroup),
    // then the rotation of each (even, odd) row pair by the angle at pos.
    if (head_w) {
#pragma unroll
      for (int j = 0; j < kOutPerLane; ++j) {
        float sq = val[j] * val[j];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) sq += __shfl_xor(sq, off, 64);
        if ((tid & 63) == 0) wsum[(j * kBlock + tid) >> 6] = sq;
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < kOutPerLane; ++j) {
        const int o = tid + j * kBlock;
        const int f0 = ((o / hd) * hd) >> 6;
        float t = 0.0f;
        if (o < HT)
          for (int f = f0; f < f0 + (hd >> 6); ++f) t += wsum[f];
        val[j] *= rsqrtf(t / (float)hd + a.head_eps) * hw[j];
      }
    }
    if (P.rope) {
#pragma unroll
      for (int j = 0; j < kOutPerLane; ++j) {
        const float partner = __shfl_xor(val[j], 1, 64);
        val[j] = (tid & 1) == 0 ? val[j] * cs[j].x - partner * cs[j].y : val[j] * cs[j].x + partner * cs[j].y;
      }
    }
  }

  T* __restrict__ out = static_cast<T*>(P.out);
#pragma unroll
  for (int j = 0; j < kOutPerLane; ++j) {
    const int o = tid + j * kBlock;
    const int r = tile * HT + o;
    if (o < HT && r < h && pos_ok) {
      long long off = r;
      if (head_layout)
        off = (long long)(r / hd) * P.head_stride + (long long)(r % hd) * P.elem_stride + pos * P.pos_stride;
      out[off] = E::from_f32(val[j] + rv[j]);
    }
  }
  if (a.splits > 1 && tid == 0) {
    __hip_atomic_store(&tickets[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}


// ---------------------------------------------------------------------------
// Configuration tables (static; no runtime autotuning).
// ---------------------------------------------------------------------------
typedef void (*KernelFn)(Args);

struct Config {
  int th;       // lanes along the output rows (tile = 8*th rows)
  int u;        // rows per lane per chunk
  bool nt;      // non-temporal weight loads
  int nmat;     // 1: plain / grouped GEMV; 2: gate/up pair with SiLU*mul
  KernelFn fn[3][4];  // [dtype][gather width: 256, 512, 1024, 2048 columns per split]
};

#define NM_CFG_G(DT, TH, U, NT, NM)                                                 \
  {&nm_gemv_kernel<DT, TH, U, 1, NT, NM>, &nm_gemv_kernel<DT, TH, U, 2, NT, NM>,     \
   &nm_gemv_kernel<DT, TH, U, 4, NT, NM>, &nm_gemv_kernel<DT, TH, U, 8, NT, NM>}
#define NM_CFG(TH, U, NT, NM)                                                       \
  {TH, U, NT, NM,                                                                   \
   {NM_CFG_G(NM_DTYPE_F16, TH, U, NT, NM), NM_CFG_G(NM_DTYPE_BF16, TH, U, NT, NM), \
    NM_CFG_G(NM_DTYPE_F32, TH, U, NT, NM)}}

// Plain / grouped GEMV configurations (ids 0..12, stable).
const Config kConfigs[] = {
    NM_CFG(16, 4, true, 1),   // 0: tile 128,  chunk 64
    NM_CFG(16, 8, true, 1),   // 1: tile 128,  chunk 128
    NM_CFG(32, 4, true, 1),   // 2: tile 256,  chunk 32
    NM_CFG(32, 8, true, 1),   // 3: tile 256,  chunk 64
    NM_CFG(32, 16, true, 1),  // 4: tile 256,  chunk 128
    NM_CFG(64, 4, true, 1),   // 5: tile 512,  chunk 16
    NM_CFG(64, 8, true, 1),   // 6: tile 512,  chunk 32
    NM_CFG(64, 16, true, 1),  // 7: tile 512,  chunk 64
    NM_CFG(128, 8, true, 1),  // 8: tile 1024, chunk 16
    NM_CFG(256, 8, true, 1),  // 9: tile 2048, chunk 8
    NM_CFG(16, 8, false, 1),  // 10: as 1, cached loads
    NM_CFG(32, 8, false, 1),  // 11: as 3, cached loads
    NM_CFG(64, 8, false, 1),  // 12: as 6, cached loads
};
constexpr int kNumConfigs = sizeof(kConfigs) / sizeof(kConfigs[0]);

// Gate/up pair configurations (each lane streams both matrices).
const Config kDualConfigs[] = {
    NM_CFG(16, 4, true, 2),   // 0: tile 128, chunk 64
    NM_CFG(32, 4, true, 2),   // 1: tile 256, chunk 32
    NM_CFG(16, 8, true, 2),   // 2: tile 128, chunk 128
    NM_CFG(32, 8, true, 2),   // 3: tile 256, chunk 64
};
constexpr int kNumDualConfigs = sizeof(kDualConfigs) / sizeof(kDualConfigs[0]);

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

// The library's own choice of configuration, from rocprof / hipGraph sweeps on
// MI355X at the Llama-3.1-8B decode shapes: 256-row tiles for wide outputs,
// 128-row tiles otherwise (h_total: summed output width of the launch).
int auto_config(int h_total, int nmat) {
  if (nmat == 2) return h_total >= 8192 ? 1 : 0;
  return h_total >= 8192 ? 3 : 1;
}

// Default split count: about 8 splits of the compressed columns per tile. The
// sweeps show the cost of a split-K handoff (one partial publish, one arrival
// atomic on a per-tile counter, one reduction) grows faster with the split
// count than the extra parallelism pays back; 8 splits of 256+ columns keep
// 64-900 workgroups streaming for every decode shape.
constexpr int kDefaultSplits = 8;

// Plan a launch of `nprob` problems (widths hs[]) sharing w, nnz, m, with
// `nmat` matrices per workgroup. The workspace holds the counters of every
// problem in its first NM_TICKET_BYTES and then nmat * splits * h floats of
// partial sums per problem.
int make_plan(int nprob, const int* hs, int w, int nnz, int m, int nmat, int cfg, int splits, Plan* p) {
  if (nprob < 1 || nprob > kMaxProblems || (nmat == 2 && nprob != 1)) return NM_ERR_BAD_SHAPE;
  long long h_total = 0;
  for (int i = 0; i < nprob; ++i) {
    const int rc = validate_shape(hs[i], w, nnz, m);
    if (rc != NM_OK) return rc;
    h_total += hs[i];
  }
  const int ncfg = nmat == 2 ? kNumDualConfigs : kNumConfigs;
  if (cfg < 0) cfg = auto_config((int)(h_total > 0x7fffffff ? 0x7fffffff : h_total), nmat);
  if (cfg >= ncfg) return NM_ERR_BAD_CONFIG;
  const Config& c = nmat == 2 ? kDualConfigs[cfg] : kConfigs[cfg];
  const int HT = c.th * kVec;
  const int CH = (kBlock / c.th) * c.u;
  if (splits <= 0) splits = kDefaultSplits;
  if (splits > w) splits = w;
  int rows = ceil_div(ceil_div(w, splits), CH) * CH;
  if (rows > kMaxRows) rows = kMaxRows;
  if (rows < CH) rows = CH;
  splits = ceil_div(w, rows);
  p->cfg = cfg;
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
    if (splits > 1) bytes += (size_t)nmat * (size_t)splits * (size_t)hs[i] * sizeof(float);
  }
  if (tickets > (size_t)kMaxTickets || blocks > 0x7fffffffLL) return NM_ERR_BAD_SHAPE;
  p->blocks = (int)blocks;
  p->workspace = bytes;
  return NM_OK;
}

// Validate a launch descriptor, plan it and launch. Every entry point of the
// C ABI goes through here.
int launch(const nm_gemv_launch_desc& d, void* workspace, size_t workspace_bytes, void* stream,
           size_t* workspace_needed) {
  if (d.dtype < NM_DTYPE_F16 || d.dtype > NM_DTYPE_F32) return NM_ERR_BAD_CONFIG;
  if (d.kind != NM_KIND_GROUPED && d.kind != NM_KIND_GATE_UP) return NM_ERR_BAD_CONFIG;
  const bool pair = d.kind == NM_KIND_GATE_UP;
  const int nmat = pair ? 2 : 1;
  const int nprob = pair ? 1 : d.nprob;  // output problems
  if (pair ? d.nprob != 2 : (d.nprob < 1 || d.nprob > kMaxProblems)) return NM_ERR_BAD_SHAPE;
  int hs[kMaxProblems];
  for (int i = 0; i < nprob; ++i) hs[i] = d.prob[i].h;
  if (pair && d.prob[1].h != d.prob[0].h) return NM_ERR_BAD_SHAPE;
  Plan p;
  int rc = make_plan(nprob, hs, d.w, d.nnz, d.m, nmat, d.config_id, d.splits, &p);
  if (rc != NM_OK) return rc;
  if (workspace_needed) {
    *workspace_needed = p.workspace;
    return NM_OK;
  }
  if (!d.vec || !workspace) return NM_ERR_NULL_POINTER;
  for (int i = 0; i < d.nprob; ++i)
    if (!d.prob[i].mat_data || !d.prob[i].mat_index) return NM_ERR_NULL_POINTER;
  for (int i = 0; i < nprob; ++i)
    if (!d.prob[i].out) return NM_ERR_NULL_POINTER;
  if (d.vec_stride < 1) return NM_ERR_BAD_SHAPE;
  for (int i = 0; i < d.nprob; ++i)
    if (((uintptr_t)d.prob[i].mat_data & 15u) != 0) return NM_ERR_MISALIGNED;
  for (int i = 0; i < nprob; ++i)
    if (((uintptr_t)d.prob[i].out & 15u) != 0) return NM_ERR_MISALIGNED;
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
  hipLaunchKernelGGL(c.fn[d.dtype][gather_slot(p.rows_per_split)], dim3(p.blocks), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), a);
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

}  // namespace

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

int nm_gemv_launch(const nm_gemv_launch_desc* desc, void* workspace, size_t workspace_bytes, void* stream) {
  if (!desc) return NM_ERR_NULL_POINTER;
  return launch(*desc, workspace, workspace_bytes, stream, nullptr);
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
    case NM_ERR_BAD_EPILOGUE:
      return "input-norm / residual / head-layout arguments rejected (contiguous 16-byte aligned vec for the "
             "norm; head_dim a multiple of 64 dividing h and the tile; pos and rope table when used)";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "unknown status code";
}

int nm_abi_version(void) { return kAbiVersion; }

}  // extern "C"
