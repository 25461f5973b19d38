// nm_gemv_kernel.h — device side of the shared-mask N:M sparse GEMV for
// MI355X (gfx950, CDNA4): element types, launch arguments and the kernel
// template. Instantiated per element type by nm_gemv_inst.hip (compiled once
// per dtype, in parallel); the host side and C ABI are in nm_gemv.hip.
//
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
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include "../../include/nmsparse_hip.h"

namespace nm_hip {

constexpr int kBlock = 256;        // lanes per workgroup
constexpr int kVec = 8;            // output rows per lane
constexpr int kMaxRows = 2048;     // compressed columns per split (LDS gather bound)
constexpr int kMaxTickets = NM_TICKET_BYTES / 4;
constexpr int kAbiVersion = 12;

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
  // Split-K carry between two launches of a decoder chain (null when unused).
  // A producer (one plain GEMV) leaves its fp32 split partials [splits, h] in
  // carry_out and writes nothing else. A consumer (CARRY) takes as its input
  // vector round_T(sum_s carry_in[s, :] + vec), the producer's epilogue with
  // vec as the residual, writes that vector to vec_out and runs as usual.
  float* carry_out;
  const float* carry_in;     // [carry_splits, K]
  void* vec_out;             // [K]
  float* ssq_slots;          // [grid] per-workgroup sums of squares of its input slice
  int carry_splits;
  // Accumulated carry (the reference's relaxed fp32 atomic accumulation,
  // triton_spmv.py:209-214, as the medium between two launches; the sums'
  // order, hence their last bits, then varies from run to run):
  //  * carry_acc with a plain producer: every split adds its partial tile
  //    into carry_out[0, :] (fp32 atomic add, agent scope) instead of
  //    writing its own row, so a consumer reads one row (carry_splits = 1);
  //  * carry_acc with the gate/up pair (carry_out set): the pair ends after
  //    its tile reduction, adding gate's and up's raw sums (without the input
  //    norm's scale) into carry_out[0, h) and [h, 2h), and storing its input's
  //    sum of squares in carry_out[2h + split] (with a carried input each
  //    split's share; otherwise the whole sum, split 0 only);
  //  * silu_in (a plain GEMV): the input is x[k] = round_T(silu(s G[k]) *
  //    (s U[k])) with G = silu_in[0, K), U = silu_in[K, 2K) and s =
  //    rsqrt(sum(silu_in[2K, 2K + silu_ssq_n)) / silu_k + silu_eps), or 1 when
  //    silu_ssq_n == 0: the pair's epilogue, done where its output is read;
  //  * zero_buf: zero_len floats this launch clears (an accumulator a later
  //    launch adds into; the launches between them order the two).
  int carry_acc;
  float* zero_buf;
  int zero_len;
  const float* silu_in;
  int silu_ssq_n;
  int silu_k;
  float silu_eps;
};

// Most producer splits a consumer reads (their partials are requested at once).
constexpr int kMaxCarry = 16;

// silu(g) = g / (1 + e^-g), with e^-g = 2^(-g log2 e) on the hardware's
// exp2 and reciprocal (v_exp_f32, v_rcp_f32; about 1 ulp each, far below the
// 16-bit rounding that follows). The IEEE expf and division took ~40
// instructions per value, in front of the first multiply where down_proj
// forms the SiLU product as it gathers.
__device__ inline float silu(float g) {
  constexpr float kLog2e = 1.44269504088896340736f;
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * kLog2e));
}

// Lane exchange inside each group of 4 lanes (DPP quad_perm): lane i reads
// lane i ^ 1 (0xB1) or i ^ 2 (0x4E). No LDS round trip.
template <int CTRL>
__device__ inline float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes of a wavefront (all lanes active), the same value
// returned to every lane, in a fixed order: quads, then half rows and rows
// (DPP row_half_mirror 0x141, row_mirror 0x140), then the four rows.
__device__ inline float wave_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  const int b = __builtin_bit_cast(int, v);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}

// Sum of squares of the elements in a 16-byte word (invalid words count 0).
template <int DT>
__device__ inline float word_ssq(const u32x4 raw, bool ok, float acc) {
  float f[8];
  if constexpr (Elem<DT>::kWords == 1) {
    const u32x4 one[1] = {raw};
    Elem<DT>::unpack(one, f);
  } else {
    const uint32_t d[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = __uint_as_float(d[e]);
#pragma unroll
    for (int e = 4; e < 8; ++e) f[e] = 0.0f;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float fe = ok ? f[e] : 0.0f;
    acc = __builtin_fmaf(fe, fe, acc);
  }
  return acc;
}

// NMAT == 1: each workgroup computes one tile/split of one problem (a plain
// GEMV when nprob == 1, several GEMVs sharing x in one grid otherwise).
// NMAT == 2: each workgroup streams the same tile/split of prob[0] (gate) and
// prob[1] (up), both of width prob[0].h, and the output prob[0].out receives
// silu(gate) * up, computed in fp32 and rounded once.
// CARRY > 0 (with NORM, at most 512 compressed columns per split, whole
// groups per split, at most CARRY producer splits): the input vector is
// finished from the previous launch's split partials (Args::carry_in). Each workgroup builds only the slice of K its
// columns read, [k0, k0 + kn), in LDS, and its sum of squares; the tile's
// last arrival adds the slices' sums in split order for the input norm.
//
// The gate/up pair kernels may use up to half the register file per lane (at
// most 2 waves per SIMD, i.e. two workgroups per CU at once, as many as the
// library's pair plans place): left to its occupancy heuristics the compiler fits the pair without
// the input norm into 135 registers, too few to keep both weight chunks of
// U = 8 rows in flight, and that kernel then ran 25-35% slower than the same
// pair with the norm (Qwen3-14B 45.3 against 34.1 us, Qwen3-32B 61.5 against
// 45.7); with the bound both fit, and both run alike.
template <int DT, int TH, int U, int G, bool NT, int NMAT, bool NORM, int CARRY, bool SILU>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(1, NMAT == 2 ? 2 : 8)))
void nm_gemv_kernel(Args a) {
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
  static_assert(!CARRY || (NORM && G <= 2 && CARRY <= kMaxCarry),
                "a carried input comes with the input norm, <= 512 columns per split");
  static_assert(!SILU || (NMAT == 1 && !NORM && !CARRY), "the SiLU-product input feeds a plain GEMV");

  constexpr int kWaves = kBlock / 64;
  constexpr int kOutPerLane = (HT + kBlock - 1) / kBlock;
  // Carried input: a slice of at most kCarryLen positions of K, four adjacent
  // ones per lane (a split of 512 columns at half density).
  constexpr int kCarryLen = 4 * kBlock;
  typedef T t4 __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(16))) float xs[NMAT][XR];
  __shared__ __attribute__((aligned(16))) float red[NMAT][TK * HT];
  __shared__ __attribute__((aligned(16))) float hs[CARRY ? kCarryLen : 4];  // slice of x * g
  __shared__ float wsum[kOutPerLane * kWaves];  // per-wave sums of the head norms
  __shared__ float nsum[kWaves];                // per-wave sums of the input norm
  __shared__ int is_last;

  // Problem of this workgroup (uniform; at most kMaxProblems entries).
  int p = 0;
  if (NMAT == 1) {
#pragma unroll
    for (int q = 1; q < kMaxProblems; ++q)
      if (q < a.nprob && (int)blockIdx.x >= a.prob[q].block_begin) p = q;
  }
  const Problem& P = a.prob[p];
  const int h = P.h;
  const int tiles = P.tiles;
  const int local = (int)blockIdx.x - P.block_begin;
  // The decode position is read at the start although only the epilogue uses
  // it, so that its latency is hidden behind the weight stream.
  const bool need_pos = P.rope != 0 || P.pos_stride != 0;
  long long pos = 0;
  if (need_pos) pos = *a.pos;

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

  // 1b. Carried input: the split's columns are whole groups (c0 and cw are
  //     multiples of nnz; the host checks), so they read the slice
  //     [k0, k0 + kn) of K, and the splits' slices partition K. Every producer
  //     split's partial (at most CARRY, addresses clamped to the last), the
  //     residual and the norm weight at four adjacent positions per lane
  //     (16-byte loads of the partials), requested before the first weight
  //     chunk so that they do not wait behind it (vmcnt is in order).
  const int k0 = CARRY ? (c0 / a.nnz) * a.m : 0;
  const int kn = CARRY ? (cw / a.nnz) * a.m : 4;  // a multiple of 4 (m is; host check), <= kCarryLen
  float4 cpart[CARRY ? CARRY : 1];
  t4 cres, cgw;
  if constexpr (CARRY > 0) {
    const int kc = k0 + min(4 * tid, kn - 4);
#pragma unroll
    for (int s = 0; s < CARRY; ++s) {
      const int ss = min(s, a.carry_splits - 1);
      cpart[s] = *reinterpret_cast<const float4*>(a.carry_in + (size_t)ss * (size_t)a.K + (size_t)kc);
    }
    cres = *reinterpret_cast<const t4*>(static_cast<const T*>(a.vec) + kc);
    cgw = *reinterpret_cast<const t4*>(static_cast<const T*>(a.norm_w) + kc);
  }

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
  // Keep the scheduler from moving the activation gather (which must wait
  // for the position loads) ahead of the first chunk's weight requests, and
  // wait for all position loads at once (vmcnt counts in issue order: only
  // the chunk's NMAT * U * W weight loads may stay outstanding).
  __builtin_amdgcn_sched_barrier(0);
  constexpr int kChunkLoads = NMAT * U * W;
  static_assert(kChunkLoads < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((kChunkLoads & 15) | (((kChunkLoads >> 4) & 3) << 14) | (7 << 4) | (15 << 8));

  // 3. Gather the activations: vec[(c/nnz)*m + position], fp32 in LDS. Rows
  //    past the split and positions outside vec read as zero.
  //    With an input RMSNorm, rmsnorm(x) = s * (x * g) with the scalar
  //    s = 1 / sqrt(mean(x^2) + eps): the gather reads x * g and s scales the
  //    finished sums. Every load here is unconditional (vec stands in for the
  //    norm weights, and mat_data for vec's words, when there is no norm; the
  //    values are then ignored): a load inside a branch makes the compiler
  //    wait at the branch's end for every load in flight, weights included.
  const T* __restrict__ gx = static_cast<const T*>(a.norm_w);
  T graw[NMAT][G];
  T wraw[NMAT][G];
  bool gok[NMAT][G];
  float sg[SILU ? G : 1], su[SILU ? G : 1];  // SILU: the pair's raw gate and up sums at the gathered positions
#pragma unroll
  for (int q = 0; q < NMAT; ++q)
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int t = tid + j * kBlock;
      const int c = c0 + min(t, cw - 1);
      const int pos = (c / a.nnz) * a.m + gidx[q][j];
      gok[q][j] = (t < cw) && (pos < a.K);
      if constexpr (CARRY) {
        graw[q][j] = 0;
        wraw[q][j] = 0;
      } else if constexpr (SILU) {
        const int pc = gok[q][j] ? pos : 0;
        sg[j] = a.silu_in[pc];
        su[j] = a.silu_in[a.K + pc];
      } else {
        graw[q][j] = vx[(long long)(gok[q][j] ? pos : 0) * a.vec_stride];
        if constexpr (NORM) wraw[q][j] = gx[gok[q][j] ? pos : 0];
      }
    }
  // SiLU-product input: the producer's sums of squares (one per lane, summed
  // in slot order below).
  float sq_slot = 0.0f;
  if constexpr (SILU) sq_slot = a.silu_ssq_n > 0 ? a.silu_in[2 * a.K + min(tid & 63, a.silu_ssq_n - 1)] : 0.0f;
  // The words of vec for mean(x^2) (contiguous, 16-byte aligned, K * size a
  // multiple of 16 with a norm; the host checks) are requested now and
  // summed after the main loop, so they never delay the weight stream.
  constexpr int kSsqWords = (NORM && !CARRY) ? 3 : 1;  // per lane: K * sizeof(T) <= 12 KiB in flight
  const u32x4* __restrict__ xw = static_cast<const u32x4*>(a.vec);
  const int nw = (int)(((long long)a.K * (long long)sizeof(T)) / 16);
  u32x4 sraw[kSsqWords];
  if constexpr (NORM && !CARRY) {
#pragma unroll
    for (int i = 0; i < kSsqWords; ++i) sraw[i] = xw[min(i * kBlock + tid, nw - 1)];
  }
  // Carried input: finish the slice, x = round_T(sum of the producer's
  // partials in split order + residual) -- the producer's own epilogue, so x
  // is bit-identical to what it would have written --, keep x * g in LDS and
  // sum x^2 over the slice. The first tile's workgroups of each split write
  // their slice of x to vec_out.
  float ssq_carry = 0.0f;
  if constexpr (CARRY) {
    float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < (CARRY ? CARRY : 1); ++s) {
      if (s < a.carry_splits) {
        sum[0] += cpart[s].x;
        sum[1] += cpart[s].y;
        sum[2] += cpart[s].z;
        sum[3] += cpart[s].w;
      }
    }
    const int kl = 4 * tid;
    if (kl < kn) {
      t4 hv;
      float4 xg;
      float f[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hv[e] = E::from_f32(sum[e] + E::to_f32(cres[e]));
        f[e] = E::to_f32(hv[e]);
        ssq_carry = __builtin_fmaf(f[e], f[e], ssq_carry);
      }
      xg.x = f[0] * E::to_f32(cgw[0]);
      xg.y = f[1] * E::to_f32(cgw[1]);
      xg.z = f[2] * E::to_f32(cgw[2]);
      xg.w = f[3] * E::to_f32(cgw[3]);
      *reinterpret_cast<float4*>(&hs[kl]) = xg;
      if (p == 0 && tile == 0) *reinterpret_cast<t4*>(static_cast<T*>(a.vec_out) + k0 + kl) = hv;
    }
  }
  // Single-matrix launches request chunk 1 here, behind the gather: the
  // barrier below then waits for chunk 0 and the gather only, and chunk 1
  // arrives during chunk 0's FMAs (a one-chunk split re-reads its last row).
  // The gate/up pair keeps chunk 1 after the barrier, which measured faster
  // for its two weight streams.
  constexpr bool kEarlyChunk1 = NMAT == 1;
  if constexpr (kEarlyChunk1) load_chunk(bufB, 1);
  __builtin_amdgcn_sched_barrier(0);  // every gather request before the first use of one
  if constexpr (CARRY) __syncthreads();  // the slice is in LDS
  float s_silu = 1.0f;
  if constexpr (SILU) {
    if (a.silu_ssq_n > 0) {
      const int b = __builtin_bit_cast(int, sq_slot);
      float t = 0.0f;
      for (int i = 0; i < a.silu_ssq_n; ++i) t += __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, i));
      s_silu = rsqrtf(t / (float)a.silu_k + a.silu_eps);
    }
  }
#pragma unroll
  for (int q = 0; q < NMAT; ++q)
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if constexpr (CARRY) {
        const int t = tid + j * kBlock;
        const int cl = min(t, cw - 1);  // column within the split
        const int li = (cl / a.nnz) * a.m + gidx[q][j];  // < kn for positions below m
        xs[q][t] = (gok[q][j] && li < kn) ? hs[li] : 0.0f;
      } else if constexpr (SILU) {
        // the pair's epilogue: silu(s g) * (s u) in fp32, one rounding to T
        const float xv = E::to_f32(E::from_f32(silu(sg[j] * s_silu) * (su[j] * s_silu)));
        xs[q][tid + j * kBlock] = gok[q][j] ? xv : 0.0f;
      } else {
        const float xv = gok[q][j] ? E::to_f32(graw[q][j]) : 0.0f;
        if constexpr (NORM) {
          xs[q][tid + j * kBlock] = xv * E::to_f32(wraw[q][j]);
        } else {
          xs[q][tid + j * kBlock] = xv;
        }
      }
    }
  __syncthreads();

  float acc[NMAT][kVec];
#pragma unroll
  for (int q = 0; q < NMAT; ++q)
#pragma unroll
    for (int e = 0; e < kVec; ++e) acc[q][e] = 0.0f;

  // FMA one chunk. Only the split's last chunk can hold rows past its end
  // (rows_per_split is a multiple of the chunk), and only there (`masked`)
  // are those rows zeroed so they contribute exactly nothing. A select on
  // the loaded words of every chunk would let the compiler hoist the selects
  // of both buffers, and with them a wait for every load in flight, to the
  // top of the loop.
  auto fma_chunk = [&](const u32x4 (&src)[NMAT][U][W], int k, bool masked) {
    const int r0 = k * CH + tk * U;
#pragma unroll
    for (int q = 0; q < NMAT; ++q) {
#pragma unroll
      for (int u4 = 0; u4 < U / 4; ++u4) {
        const float4 xv = *reinterpret_cast<const float4*>(&xs[q][r0 + 4 * u4]);
        const float xq[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bool ok = !masked || (r0 + 4 * u4 + s) < cw;
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
  //    chunk k is consumed. Loads inside the loop are unconditional. For
  //    single-matrix launches, scheduling barriers keep each refill right
  //    behind the FMAs that free its buffer, ahead of the next chunk's FMAs
  //    (down -4.5%, o -1.5%); the gate/up pair measured the same or slower
  //    with them.
  constexpr bool kPinOrder = NMAT == 1;
  int k = 0;
  if constexpr (kEarlyChunk1) {
    // Chunks k and k+1 are in flight on entry; each buffer is refilled as
    // soon as it has been consumed (past the split's end the clamped rows
    // are re-read and never used).
    for (; k + 2 < nch; k += 2) {
      fma_chunk(bufA, k, false);
      if constexpr (kPinOrder) __builtin_amdgcn_sched_barrier(0);
      load_chunk(bufA, k + 2);
      if constexpr (kPinOrder) __builtin_amdgcn_sched_barrier(0);
      fma_chunk(bufB, k + 1, false);
      if constexpr (kPinOrder) __builtin_amdgcn_sched_barrier(0);
      load_chunk(bufB, k + 3);
      if constexpr (kPinOrder) __builtin_amdgcn_sched_barrier(0);
    }
    fma_chunk(bufA, k, true);
    if (k + 1 < nch) fma_chunk(bufB, k + 1, true);
  } else {
    for (; k + 2 < nch; k += 2) {
      load_chunk(bufB, k + 1);
      if constexpr (kPinOrder) __builtin_amdgcn_sched_barrier(0);
      fma_chunk(bufA, k, false);
      if constexpr (kPinOrder) __builtin_amdgcn_sched_barrier(0);
      load_chunk(bufA, k + 2);
      if constexpr (kPinOrder) __builtin_amdgcn_sched_barrier(0);
      fma_chunk(bufB, k + 1, false);
      if constexpr (kPinOrder) __builtin_amdgcn_sched_barrier(0);
    }
    if (k + 1 < nch) {
      load_chunk(bufB, k + 1);
      fma_chunk(bufA, k, true);
      fma_chunk(bufB, k + 1, true);
    } else {
      fma_chunk(bufA, k, true);
    }
  }

  // 4b. An accumulator a later launch adds into is cleared here, behind the
  //     weight stream (its stores would otherwise hold up the first waits):
  //     workgroup b clears its share of zero_len floats (16-byte stores).
  if (a.zero_buf != nullptr) {
    const int per = (((a.zero_len + (int)gridDim.x - 1) / (int)gridDim.x) + 3) & ~3;
    const int z0 = (int)blockIdx.x * per;
    const int z1 = min(z0 + per, a.zero_len);
    for (int i = z0 + 4 * tid; i < z1; i += 4 * kBlock)
      *reinterpret_cast<float4*>(a.zero_buf + i) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }

  // 5. Reduce the TK lane-rows of the tile through LDS (fixed order), and
  //    the input norm's sum of squares (fixed order too).
#pragma unroll
  for (int q = 0; q < NMAT; ++q) {
    float4* rp = reinterpret_cast<float4*>(&red[q][tk * HT + th * kVec]);
    rp[0] = make_float4(acc[q][0], acc[q][1], acc[q][2], acc[q][3]);
    rp[1] = make_float4(acc[q][4], acc[q][5], acc[q][6], acc[q][7]);
  }
  if constexpr (NORM) {
    float ssq = 0.0f;
    if constexpr (CARRY) {
      ssq = ssq_carry;
    } else {
#pragma unroll
      for (int i = 0; i < kSsqWords; ++i) ssq = word_ssq<DT>(sraw[i], i * kBlock + tid < nw, ssq);
      for (int base = kSsqWords * kBlock; base < nw; base += kBlock)  // K * sizeof(T) > 12 KiB only
        ssq = word_ssq<DT>(xw[min(base + tid, nw - 1)], base + tid < nw, ssq);
    }
    ssq = wave_sum(ssq);
    if ((tid & 63) == 0) nsum[tid >> 6] = ssq;
  }
  __syncthreads();
  float s_in = 1.0f;
  float slice_ssq = 0.0f;  // CARRY: this split's share of sum(x^2)
  if constexpr (NORM) {
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) t += nsum[i];
    slice_ssq = t;
    if (!CARRY || a.splits == 1) s_in = rsqrtf(t / (float)a.K + a.norm_eps);
  }

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

  // A producer leaves its partial tile for the next launch (which reads it
  // after this grid has completed) and is done: no handoff, no epilogue.
  if constexpr (NMAT == 1 && !CARRY) {
    if (a.carry_out != nullptr) {
      if (a.carry_acc) {  // accumulated: every split adds into row 0
#pragma unroll
        for (int j = 0; j < kOutPerLane; ++j) {
          const int o = tid + j * kBlock;
          const int r = tile * HT + o;
          if (o < HT && r < h)
            (void)__hip_atomic_fetch_add(a.carry_out + r, tsum[0][j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
      }
      float* part = a.carry_out + (size_t)split * (size_t)h;
#pragma unroll
      for (int j = 0; j < kOutPerLane; ++j) {
        const int o = tid + j * kBlock;
        const int r = tile * HT + o;
        if (o < HT && r < h) part[r] = tsum[0][j];
      }
      return;
    }
  }
  // The gate/up pair as an accumulated producer: its raw sums go to the
  // consumer (which applies the input norm's scale and the SiLU product when
  // it gathers them), the input's sum of squares to slot 2h + split; no
  // handoff, no epilogue.
  if constexpr (NMAT == 2) {
    if (a.carry_out != nullptr) {
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int j = 0; j < kOutPerLane; ++j) {
          const int o = tid + j * kBlock;
          const int r = tile * HT + o;
          if (o < HT && r < h)
            (void)__hip_atomic_fetch_add(a.carry_out + (size_t)q * (size_t)h + r, tsum[q][j], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
        }
      if constexpr (NORM) {
        if (tid == 0 && tile == 0 && (CARRY || split == 0))
          (void)__hip_atomic_exchange(a.carry_out + 2 * (size_t)h + split, slice_ssq, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
      }
      return;
    }
  }

  uint32_t* tickets = P.tickets;
  if (a.splits > 1) {
    // 6. Split-K: publish the partial tile, count arrivals, last one reduces.
    //    The handoff uses agent-scope atomics only, never an agent-scope
    //    fence: on gfx950 such a fence writes back and invalidates the whole
    //    L2 of the workgroup's XCD (buffer_wbl2 / buffer_inv), which costs
    //    more than the GEMV itself, and exists to make non-atomic data
    //    coherent; every word shared here is written and read by agent-scope
    //    atomics. Each partial is published with an agent-scope atomic swap
    //    (relaxed, result unused: the no-return global_atomic_swap, performed
    //    at the agent's coherence point like every agent-scope RMW), and each
    //    lane waits for the completion of all of them (vmcnt counts
    //    no-return atomics on gfx9-family GPUs) before the barrier. Lane 0
    //    then counts the arrival (a returning agent-scope add); the last
    //    arrival, ordered after its add's returned value, reads every partial
    //    with agent-scope atomic loads (sc1) in split order, so the sum is
    //    deterministic.
#pragma unroll
    for (int q = 0; q < NMAT; ++q) {
      float* part = a.prob[NMAT == 1 ? p : q].partial + (size_t)split * (size_t)h;
#pragma unroll
      for (int j = 0; j < kOutPerLane; ++j) {
        const int o = tid + j * kBlock;
        const int r = tile * HT + o;
        if (o < HT && r < h)
          (void)__hip_atomic_exchange(part + r, tsum[q][j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if constexpr (CARRY) {
      if (tid == 0)
        (void)__hip_atomic_exchange(a.ssq_slots + blockIdx.x, slice_ssq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
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
    // The partials of a group of 8 splits are read for every matrix and
    // output of the lane at once (one round trip per group, not one per
    // matrix); each output sums them in split order. Lanes past the tile
    // read the tile's last column (clamped) and keep their sums unused.
    float sacc[NMAT][kOutPerLane];
    const float* pp[NMAT][kOutPerLane];
#pragma unroll
    for (int q = 0; q < NMAT; ++q)
#pragma unroll
      for (int j = 0; j < kOutPerLane; ++j) {
        const int r = min(tile * HT + min(tid + j * kBlock, HT - 1), h - 1);
        pp[q][j] = a.prob[NMAT == 1 ? p : q].partial + r;
        sacc[q][j] = 0.0f;
      }
    // CARRY: the splits' slice sums of squares (slot of the workgroup of
    // split s = its grid index) are read in the same round trip, summed in
    // split order.
    const float* slot = CARRY ? a.ssq_slots + P.block_begin + tile : nullptr;
    float ssq_all = 0.0f;
    int sp = 0;
    for (; sp + 8 <= a.splits; sp += 8) {
      float t8[NMAT][kOutPerLane][8];
      float n8[8];
#pragma unroll
      for (int q = 0; q < NMAT; ++q)
#pragma unroll
        for (int j = 0; j < kOutPerLane; ++j)
#pragma unroll
          for (int i = 0; i < 8; ++i)
            t8[q][j][i] = __hip_atomic_load(pp[q][j] + (size_t)(sp + i) * (size_t)h, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
      if constexpr (CARRY) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          n8[i] = __hip_atomic_load(slot + (size_t)(sp + i) * (size_t)tiles, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int q = 0; q < NMAT; ++q)
#pragma unroll
        for (int j = 0; j < kOutPerLane; ++j)
#pragma unroll
          for (int i = 0; i < 8; ++i) sacc[q][j] += t8[q][j][i];
      if constexpr (CARRY) {
#pragma unroll
        for (int i = 0; i < 8; ++i) ssq_all += n8[i];
      }
    }
    for (; sp < a.splits; ++sp) {
      float t1[NMAT][kOutPerLane];
      float n1 = 0.0f;
#pragma unroll
      for (int q = 0; q < NMAT; ++q)
#pragma unroll
        for (int j = 0; j < kOutPerLane; ++j)
          t1[q][j] = __hip_atomic_load(pp[q][j] + (size_t)sp * (size_t)h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if constexpr (CARRY)
        n1 = __hip_atomic_load(slot + (size_t)sp * (size_t)tiles, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int q = 0; q < NMAT; ++q)
#pragma unroll
        for (int j = 0; j < kOutPerLane; ++j) sacc[q][j] += t1[q][j];
      if constexpr (CARRY) ssq_all += n1;
    }
    if constexpr (CARRY) s_in = rsqrtf(ssq_all / (float)a.K + a.norm_eps);
#pragma unroll
    for (int q = 0; q < NMAT; ++q)
#pragma unroll
      for (int j = 0; j < kOutPerLane; ++j) tsum[q][j] = sacc[q][j];
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
        const float sq = wave_sum(val[j] * val[j]);
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
        const float partner = dpp<0xB1>(val[j]);  // row r ^ 1 is lane tid ^ 1
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
// Small-batch SpMM: out[b, r] for b < batch <= NB rows of activations that
// share the weight stream (multi-token decode, batched serving, short
// prefills). The work decomposition, FMA order, lane-row reduction and
// split-K handoff are those of nm_gemv_kernel, so with the same tile, chunk
// and split plan each output row is bit-identical to the GEMV of that row.
// ---------------------------------------------------------------------------
constexpr int kMaxBatch = 8;
constexpr int kMaxRowsSpmm = 1024;  // compressed columns per split (LDS: NB * (rows + 2048) floats)

struct SpmmArgs {
  const void* x;            // [batch, K], rows x_row_stride elements apart, unit column stride
  long long x_row_stride;
  const void* mat_data;     // [w, h]
  const uint8_t* mat_index; // [w / nnz, nnz]
  void* out;                // [batch, h], rows out_row_stride elements apart
  long long out_row_stride;
  float* partial;           // [splits, batch, h] fp32, unused when splits == 1
  uint32_t* tickets;        // [tiles] arrival counters, zero between launches
  int batch;
  int h;
  int tiles;
  int w;
  int nnz;
  int m;
  int K;
  int splits;
  int rows_per_split;
};

template <int DT, int TH, int U, int G, bool NT, int NB>
__global__ __launch_bounds__(kBlock) void nm_spmm_kernel(SpmmArgs a) {
  using E = Elem<DT>;
  typedef typename E::scalar T;
  constexpr int W = E::kWords;
  constexpr int TK = kBlock / TH;
  constexpr int HT = TH * kVec;
  constexpr int CH = TK * U;
  constexpr int XR = G * kBlock;
  constexpr int kOutPerLane = (HT + kBlock - 1) / kBlock;
  static_assert(U % 4 == 0 && XR % CH == 0, "chunk shape");
  static_assert(NB >= 1 && NB <= kMaxBatch, "batch rows per launch");

  __shared__ __attribute__((aligned(16))) float xs[NB][XR];
  __shared__ __attribute__((aligned(16))) float red[NB][TK * HT];
  __shared__ int is_last;

  const int h = a.h;
  const int tid = threadIdx.x;
  const int th = tid % TH;
  const int tk = tid / TH;
  const int tile = (int)blockIdx.x % a.tiles;
  const int split = (int)blockIdx.x / a.tiles;
  const int c0 = split * a.rows_per_split;
  const int cw = min(a.rows_per_split, a.w - c0);
  const int nch = (cw + CH - 1) / CH;
  const int col = tile * HT + th * kVec;
  const int col_ld = min(col, h - kVec);
  const T* __restrict__ md_tile = static_cast<const T*>(a.mat_data) + (size_t)c0 * (size_t)h + (size_t)col_ld;

  // 1. In-group positions, 2. the first chunk of weights, then all position
  //    loads waited for at once (see nm_gemv_kernel).
  int gidx[G];
#pragma unroll
  for (int j = 0; j < G; ++j) gidx[j] = (int)a.mat_index[c0 + min(tid + j * kBlock, cw - 1)];
  auto load_chunk = [&](u32x4 (&dst)[U][W], int k) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = min(k * CH + tk * U + u, cw - 1);
      const u32x4* ptr = reinterpret_cast<const u32x4*>(md_tile + (size_t)r * (size_t)h);
#pragma unroll
      for (int v = 0; v < W; ++v) dst[u][v] = load16<NT>(ptr + v);
    }
  };
  u32x4 bufA[U][W];
  u32x4 bufB[U][W];
  load_chunk(bufA, 0);
  __builtin_amdgcn_sched_barrier(0);
  constexpr int kAfterIdx = U * W;
  __builtin_amdgcn_s_waitcnt((kAfterIdx & 15) | (((kAfterIdx >> 4) & 3) << 14) | (7 << 4) | (15 << 8));

  // 3. Gather every batch row's activations (rows past `batch` read row
  //    batch - 1 and are zeroed) into LDS as fp32.
  int gpos[G];
  bool gok[G];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const int t = tid + j * kBlock;
    const int c = c0 + min(t, cw - 1);
    const int pos = (c / a.nnz) * a.m + gidx[j];
    gok[j] = (t < cw) && (pos < a.K);
    gpos[j] = gok[j] ? pos : 0;
  }
  T graw[NB][G];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const T* __restrict__ xb = static_cast<const T*>(a.x) + (long long)min(b, a.batch - 1) * a.x_row_stride;
#pragma unroll
    for (int j = 0; j < G; ++j) graw[b][j] = xb[gpos[j]];
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < G; ++j)
      xs[b][tid + j * kBlock] = (gok[j] && b < a.batch) ? E::to_f32(graw[b][j]) : 0.0f;
  __syncthreads();

  float acc[NB][kVec];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int e = 0; e < kVec; ++e) acc[b][e] = 0.0f;

  auto fma_chunk = [&](const u32x4 (&src)[U][W], int k, bool masked) {  // masked: as nm_gemv_kernel
    const int r0 = k * CH + tk * U;
#pragma unroll
    for (int u4 = 0; u4 < U / 4; ++u4) {
      float4 xv[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) xv[b] = *reinterpret_cast<const float4*>(&xs[b][r0 + 4 * u4]);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bool ok = !masked || (r0 + 4 * u4 + s) < cw;
        u32x4 rw[W];
#pragma unroll
        for (int v = 0; v < W; ++v) rw[v] = ok ? src[4 * u4 + s][v] : u32x4{0u, 0u, 0u, 0u};
        float wv[kVec];
        E::unpack(rw, wv);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const float xq = s == 0 ? xv[b].x : (s == 1 ? xv[b].y : (s == 2 ? xv[b].z : xv[b].w));
#pragma unroll
          for (int e = 0; e < kVec; ++e) acc[b][e] = __builtin_fmaf(wv[e], xq, acc[b][e]);
        }
      }
    }
  };

  // 4. Stream the split (as nm_gemv_kernel).
  int k = 0;
  for (; k + 2 < nch; k += 2) {
    load_chunk(bufB, k + 1);
    __builtin_amdgcn_sched_barrier(0);
    fma_chunk(bufA, k, false);
    __builtin_amdgcn_sched_barrier(0);
    load_chunk(bufA, k + 2);
    __builtin_amdgcn_sched_barrier(0);
    fma_chunk(bufB, k + 1, false);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (k + 1 < nch) {
    load_chunk(bufB, k + 1);
    fma_chunk(bufA, k, true);
    fma_chunk(bufB, k + 1, true);
  } else {
    fma_chunk(bufA, k, true);
  }

  // 5. Lane-row reduction per batch row (fixed order).
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    float4* rp = reinterpret_cast<float4*>(&red[b][tk * HT + th * kVec]);
    rp[0] = make_float4(acc[b][0], acc[b][1], acc[b][2], acc[b][3]);
    rp[1] = make_float4(acc[b][4], acc[b][5], acc[b][6], acc[b][7]);
  }
  __syncthreads();
  float tsum[NB][kOutPerLane];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < kOutPerLane; ++j) {
      const int o = tid + j * kBlock;
      float s = 0.0f;
      if (o < HT) {
#pragma unroll
        for (int t = 0; t < TK; ++t) s += red[b][t * HT + o];
      }
      tsum[b][j] = s;
    }

  // 6. Split-K handoff (as nm_gemv_kernel; partials [split, batch, h]), with
  //    one difference: the partials are published with agent-scope atomic
  //    stores (`global_store_dword ... sc1`, write-through, counted by vmcnt
  //    like the swaps) instead of atomic swaps. With NB partials per lane the
  //    swaps' read-modify-write throughput shows (batch 4-8: 2-3% slower);
  //    every shared word is still written and read by agent-scope atomics.
  if (a.splits > 1) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (b >= a.batch) break;
      float* part = a.partial + ((size_t)split * (size_t)a.batch + (size_t)b) * (size_t)h;
#pragma unroll
      for (int j = 0; j < kOutPerLane; ++j) {
        const int o = tid + j * kBlock;
        const int r = tile * HT + o;
        if (o < HT && r < h) __hip_atomic_store(part + r, tsum[b][j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(&a.tickets[tile], 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      is_last = (prev == (uint32_t)(a.splits - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (!is_last) return;
    // Partials of a group of splits read for every batch row and output at
    // once (as nm_gemv_kernel); rows >= batch read row batch - 1, unused.
    const size_t step = (size_t)a.batch * (size_t)h;
    constexpr int G8 = NB * kOutPerLane * 8 <= 32 ? 8 : 4;  // splits per group: <= 32 loads in flight per lane
    float sacc[NB][kOutPerLane];
    const float* pp[NB][kOutPerLane];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int j = 0; j < kOutPerLane; ++j) {
        const int r = min(tile * HT + min(tid + j * kBlock, HT - 1), h - 1);
        pp[b][j] = a.partial + (size_t)min(b, a.batch - 1) * (size_t)h + r;
        sacc[b][j] = 0.0f;
      }
    int sp = 0;
    for (; sp + G8 <= a.splits; sp += G8) {
      float t8[NB][kOutPerLane][8];
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int j = 0; j < kOutPerLane; ++j)
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (i < G8)
              t8[b][j][i] = __hip_atomic_load(pp[b][j] + (size_t)(sp + i) * step, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int j = 0; j < kOutPerLane; ++j)
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (i < G8) sacc[b][j] += t8[b][j][i];
    }
    for (; sp < a.splits; ++sp) {
      float t1[NB][kOutPerLane];
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int j = 0; j < kOutPerLane; ++j)
          t1[b][j] = __hip_atomic_load(pp[b][j] + (size_t)sp * step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int j = 0; j < kOutPerLane; ++j) sacc[b][j] += t1[b][j];
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int j = 0; j < kOutPerLane; ++j) tsum[b][j] = sacc[b][j];
  }

  // 7. Outputs of the finished tile.
  T* __restrict__ out = static_cast<T*>(a.out);
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b >= a.batch) break;
#pragma unroll
    for (int j = 0; j < kOutPerLane; ++j) {
      const int o = tid + j * kBlock;
      const int r = tile * HT + o;
      if (o < HT && r < h) out[(long long)b * a.out_row_stride + r] = E::from_f32(tsum[b][j]);
    }
  }
  if (a.splits > 1 && tid == 0) {
    __hip_atomic_store(&a.tickets[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------
// Kernel configurations (ids are stable; the host side keeps the metadata).
// X(TH, U, NT): lanes along the output rows (tile = 8 * TH rows), rows per lane
// per chunk, non-temporal weight loads.
// ---------------------------------------------------------------------------
#define NM_PLAIN_CONFIGS(X)                                                       \
  X(16, 4, true)   /* 0: tile 128,  chunk 64 */                                   \
  X(16, 8, true)   /* 1: tile 128,  chunk 128 */                                  \
  X(32, 4, true)   /* 2: tile 256,  chunk 32 */                                   \
  X(32, 8, true)   /* 3: tile 256,  chunk 64 */                                   \
  X(32, 16, true)  /* 4: tile 256,  chunk 128 */                                  \
  X(64, 4, true)   /* 5: tile 512,  chunk 16 */                                   \
  X(64, 8, true)   /* 6: tile 512,  chunk 32 */                                   \
  X(64, 16, true)  /* 7: tile 512,  chunk 64 */                                   \
  X(128, 8, true)  /* 8: tile 1024, chunk 16 */                                   \
  X(256, 8, true)  /* 9: tile 2048, chunk 8 */                                    \
  X(16, 8, false)  /* 10: as 1, cached loads */                                   \
  X(32, 8, false)  /* 11: as 3, cached loads */                                   \
  X(64, 8, false)  /* 12: as 6, cached loads */

// Gate/up pair configurations (each lane streams both matrices).
#define NM_PAIR_CONFIGS(X)                                                        \
  X(16, 4, true)   /* 0: tile 128, chunk 64 */                                    \
  X(32, 4, true)   /* 1: tile 256, chunk 32 */                                    \
  X(16, 8, true)   /* 2: tile 128, chunk 128 */                                   \
  X(32, 8, true)   /* 3: tile 256, chunk 64 */                                    \
  X(64, 4, true)   /* 4: tile 512, chunk 16 */                                    \
  X(64, 8, true)   /* 5: tile 512, chunk 32 */

#define NM_COUNT_CONFIG(TH, U, NT) +1
constexpr int kNumConfigs = 0 NM_PLAIN_CONFIGS(NM_COUNT_CONFIG);
constexpr int kNumDualConfigs = 0 NM_PAIR_CONFIGS(NM_COUNT_CONFIG);
#undef NM_COUNT_CONFIG

typedef void (*KernelFn)(Args);

// The kernels of one configuration and element type:
// fn[gather slot: 256, 512, 1024, 2048 columns per split][variant: plain,
// input norm, input norm with a carried input of <= 8 or <= 16 producer
// splits or of one accumulated row (slots 0-1 only, else null), the
// SiLU-product input (single-matrix configurations only, else null)].
enum Variant { kVarPlain = 0, kVarNorm, kVarCarry8, kVarCarry16, kVarCarry1, kVarSilu, kNumVariants };
struct KernelRow {
  KernelFn fn[4][kNumVariants];
};

// SpMM configurations: the plain ids 0-3 (th16/th32 x u4/u8, non-temporal).
#define NM_SPMM_CONFIGS(X) X(16, 4, true) X(16, 8, true) X(32, 4, true) X(32, 8, true)
constexpr int kNumSpmmConfigs = 4;

typedef void (*SpmmFn)(SpmmArgs);

// fn[batch rows per launch: 2, 4, 8][gather slot: 256, 512, 1024 columns per split].
struct SpmmRow {
  SpmmFn fn[3][3];
};

// Defined in nm_gemv_inst.hip, one object per element type.
extern const KernelRow kPlainKernelsF16[kNumConfigs];
extern const KernelRow kPlainKernelsBF16[kNumConfigs];
extern const KernelRow kPlainKernelsF32[kNumConfigs];
extern const KernelRow kPairKernelsF16[kNumDualConfigs];
extern const KernelRow kPairKernelsBF16[kNumDualConfigs];
extern const KernelRow kPairKernelsF32[kNumDualConfigs];
extern const SpmmRow kSpmmKernelsF16[kNumSpmmConfigs];
extern const SpmmRow kSpmmKernelsBF16[kNumSpmmConfigs];
extern const SpmmRow kSpmmKernelsF32[kNumSpmmConfigs];

}  // namespace nm_hip
