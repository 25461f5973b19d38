// nm_spmm_mc.hip — the matrix-core SpMM: out[b, :] = W x[b, :] for
// NM_MAX_BATCH < batch <= NM_MC_MAX_BATCH activation rows (prefill chunks,
// batched serving) over the shared-mask N:M packed weights, fp16 and bf16,
// on gfx950's v_mfma_f32_16x16x32_{f16,bf16}. The C ABI (nm_spmm_mc*) is
// declared in include/nmsparse_hip.h.
//
// out[b, r] = RNE_T( sum_c f32(mat_data[c, r]) * f32(x[b, (c/nnz)*m + mat_index[c]]) )
//
// is the GEMM out = Xg W of the gathered activations Xg[b, c] (batch x w)
// and the packed weights W = mat_data (w x h): the shared mask makes the
// gather one index per compressed column for every row. Past 8 rows the
// small-batch SpMM's FMAs (rows x 8 per 16-B weight word) and its one launch
// per 8 rows dominate; here each weight word is read from HBM once per
// launch and multiplied on the matrix cores for all rows.
//
//  * A first kernel gathers the activations once per call, Xg[b, c] =
//    x[b, (c/nnz)*m + mat_index[c]], into the workspace ([batch, wp], wp = w
//    rounded up to whole 64-column chunks, zero past w).
//  * The main kernel: a workgroup (256 lanes = 4 wave64) owns an output tile
//    of HT columns r and all BT >= batch rows (16, 32, 64 or 128), over one
//    split of the compressed columns c. The 4 waves split the tile into row
//    ranges (one 16-row block each up to 32 rows, two / four blocks each at
//    64 / 128) x column ranges; a wave keeps its rows x columns as 16 x 16 fp32
//    accumulator blocks in registers. Chunks of 64 compressed columns (two
//    MFMA K steps): the weight rows [64 x HT] are staged through LDS. Up to
//    1024 outputs (register-staged): loaded 16 B per lane (non-temporal),
//    two LDS buffers, the activation operands straight from Xg, two chunks
//    in flight in registers while one is multiplied. Past that (DMA): the
//    weight rows and the chunk's activation fragments go from memory into a
//    ring of LDS stages (global_load_lds_dwordx4), see the kernel.
//  * MFMA operands: the activation block is K-contiguous in Xg; the weight
//    block, stored with the outputs contiguous, is read transposed with
//    ds_read_b64_tr_b16 (lane l of a 16-lane group receives element l of
//    each of the 4 rows the group addresses, 4 consecutive elements per lane).
//  * Split-K as the small-batch SpMM: partials [split, batch, h] published
//    with agent-scope atomic stores, an agent-scope arrival counter per tile,
//    the last arrival sums the partials in split order and rounds to T.
//    Deterministic for a given plan; not bit-identical to the GEMV (the
//    matrix core's dot products have their own order).
#include "nm_gemv_kernel.h"

namespace nm_hip {
namespace {

constexpr int kMcCK = 64;         // compressed columns per chunk: two MFMA K steps of 32
constexpr int kMcNumConfigs = 6;  // output tile HT = 64, 128, 256; register-staged (0-2) or DMA (3-5) weights
static_assert(NM_MC_MAX_BATCH == 128, "batch tiles of 16, 32, 64 and 128 rows");

typedef short s4 __attribute__((ext_vector_type(4)));
typedef short s8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s4 lds_s4;

template <int DT>
__device__ inline f4 mfma16x16x32(s8 a, s8 b, f4 c);
template <>
__device__ inline f4 mfma16x16x32<NM_DTYPE_F16>(s8 a, s8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
}
template <>
__device__ inline f4 mfma16x16x32<NM_DTYPE_BF16>(s8 a, s8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, a), __builtin_bit_cast(b8, b), c, 0, 0, 0);
}

// MFMA 16x16x32 register layout (gfx950; checked on the GPU): A[16 x 32]:
// lane l holds row l % 16, K elements 8*(l/16) .. +7; B[32 x 16]: column
// l % 16, K elements 8*(l/16) .. +7; D[16 x 16]: column l % 16, rows
// 4*(l/16) .. +3.
// LDS stages of the DMA variant per tile width (S - 1 chunks of 64 x HT
// weights and their activation fragments in flight): 4 / 3 / 3 for 64- /
// 128- / 256-column tiles, fitted to graph-replay sweeps of 2-8 stages at
// 16-64 rows over the Llama-3.1-8B and Qwen3 shapes (deeper rings measured
// up to 8% slower, two stages up to 30%). At most 65 KB of LDS per
// workgroup.
constexpr int mc_stages(int ht) { return ht == 64 ? 4 : 3; }
constexpr int kMcNtAux = 2;  // cache policy of the weight DMA: non-temporal

// Inline asm with register constraints exists only in the device pass (the
// host pass of a kernel template would otherwise reject it and drop the stub).
template <int N>
__device__ inline void mc_wait_vm() {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
#endif
}

// Two transposed 16-bit reads, rows 0-3 and 4-7 of a 16-lane group (the
// second OFF bytes further), without a wait: see mc_lds_wait.
template <int OFF>
__device__ inline void mc_read_tr_pair(s4& lo, s4& hi, uint32_t addr) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("ds_read_b64_tr_b16 %0, %2\n\tds_read_b64_tr_b16 %1, %2 offset:%3"
               : "=&v"(lo), "=&v"(hi)
               : "v"(addr), "n"(OFF));
#endif
}

// One 16-B LDS read without a wait: see mc_lds_wait.
__device__ inline void mc_read_b128(s8& v, uint32_t addr) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
#endif
}

__device__ inline void mc_lds_wait() {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#endif
}

// Orders every later use of v after the preceding mc_lds_wait.
__device__ inline void mc_after_wait(s4& v) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("" : "+v"(v));
#endif
}
__device__ inline void mc_after_wait8(s8& v) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("" : "+v"(v));
#endif
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) char lds_char;

// Workgroup `block` of one product (the tile and split it owns follow from
// it); the kernels below are this for one product, or for several products
// of the same activations in one grid.
template <int DT, int BT, int HT, bool DMA>
__device__ __forceinline__ void mc_tile(const SpmmArgs& a, const int block) {
  using E = Elem<DT>;
  typedef typename E::scalar T;  // 16-bit storage
  constexpr int RBT = BT / 16;              // 16-row blocks per tile
  // Waves along the rows: one per 16-row block up to 32 rows, two of two
  // (four) blocks each at 64 (128) rows (four waves of one block each read
  // the whole weight tile from LDS four times over, and measured 2-9% slower
  // at 64 rows).
  constexpr int WM = RBT < 2 ? RBT : 2;
  constexpr int WN = 4 / WM;                // waves along the output columns
  constexpr int MB = RBT / WM;              // 16-row blocks per wave
  constexpr int NW = HT / WN;               // output columns per wave
  constexpr int NBK = NW / 16;              // 16-column blocks per wave
  constexpr int LPR = HT / 8;               // lanes per weight row (16 B each)
  constexpr int RPI = kBlock / LPR;         // weight rows per load
  constexpr int NI = kMcCK / RPI;           // weight loads per lane per chunk
  constexpr int WSTR = HT + 16;             // LDS weight row stride (elements)
  constexpr int KS = kMcCK / 32;            // MFMA K steps per chunk
  static_assert(NBK >= 1 && NI >= 1 && RPI * NI == kMcCK, "tile shape");

  constexpr int S = mc_stages(HT);           // DMA variant: LDS stages
  constexpr int RB = HT * 2;                 // DMA variant: bytes per LDS weight row (no padding)
  constexpr int SB = kMcCK * RB;             // DMA variant: weight bytes per stage
  constexpr int NFA = RBT * KS;              // DMA variant: activation fragments (1 KB) per chunk
  constexpr int NA = (NFA + 3) / 4;          // DMA variant: activation fragments each wave loads per chunk
  constexpr int SA = NFA * 1024;             // DMA variant: activation bytes per stage
  // (waves without a fragment of their own load one into a spare 1 KB that is never read)
  constexpr int kLdsBytes = DMA ? S * (SB + SA) + (4 * NA > NFA ? 1024 : 0) : 2 * kMcCK * WSTR * (int)sizeof(T);
  // The whole static LDS is the staging (the split-K tail reuses its first
  // word once every wave is past the main loop).
  __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];
  T(*ws)[kMcCK * WSTR] = reinterpret_cast<T(*)[kMcCK * WSTR]>(lds);
  int& is_last = *reinterpret_cast<int*>(lds);

  const int h = a.h;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int rb = 16 * MB * (wave % WM);  // the wave's first batch row
  const int cb = NW * (wave / WM);  // the wave's first column within the tile
  const int lg = (tid & 63) >> 4;
  const int li = tid & 15;
  const int tile = block % a.tiles;
  const int split = block / a.tiles;
  const int c0 = split * a.rows_per_split;
  const int cw = min(a.rows_per_split, a.w - c0);
  const int nch = (cw + kMcCK - 1) / kMcCK;  // c0 + nch * kMcCK <= wp (rows_per_split: whole chunks)

  // Weight rows: lane tid loads 16 B of row wrow + i * RPI of each chunk
  // (rows past the split re-read its last row and are zeroed in LDS;
  // columns past h read the last 8 columns and feed only outputs >= h).
  const T* __restrict__ md = static_cast<const T*>(a.mat_data);
  const int wrow = tid / LPR;
  const int wcol = (tid % LPR) * 8;
  const int gcol = min(tile * HT + wcol, h - 8);
  auto load_w = [&](u32x4 (&dst)[NI], int k) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int r = c0 + min(k * kMcCK + wrow + i * RPI, cw - 1);
      dst[i] = load16<true>(reinterpret_cast<const u32x4*>(md + (size_t)r * (size_t)h + gcol));
    }
  };
  // Gathered activations, stored by the gather in MFMA operand order: the A
  // operand of row block j (16 rows) for K step ks of chunk q (global chunk
  // index) is one contiguous 1 KB fragment at ((q * KS + ks) * RBK + j) * 512
  // elements, lane l's 16 B at l * 8 (row 16 j + l % 16, compressed columns
  // 64 q + 32 ks + 8 (l / 16) .. + 7; rows past the batch and columns past w
  // zero). RBK (row blocks stored) comes in x_row_stride. One wave's operand
  // load is 8 whole cache lines instead of 16 half ones of a row-major
  // [batch, w] array.
  const T* __restrict__ xg = static_cast<const T*>(a.x);
  const int rbk_n = (int)a.x_row_stride;
  const int lane = tid & 63;
  auto load_a = [&](u32x4 (&dst)[MB][KS], int k) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int rbk = min((rb >> 4) + mb, rbk_n - 1);
        const size_t frag = ((size_t)(c0 / kMcCK + k) * KS + ks) * (size_t)rbk_n + (size_t)rbk;
        dst[mb][ks] = *reinterpret_cast<const u32x4*>(xg + frag * 512 + (size_t)lane * 8);
      }
  };
  f4 acc[MB][NBK];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NBK; ++nb) acc[mb][nb] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  if constexpr (DMA) {
#if defined(__HIP_DEVICE_COMPILE__)  // device code only: the host pass needs just the kernel's stub
    // Weight chunks go from HBM straight into a ring of S LDS stages
    // (global_load_lds_dwordx4: no registers held while in flight), S - 1
    // chunks ahead of the one multiplied, and so do the activation fragments
    // of the same chunks (once per workgroup, shared by its waves), so that
    // one in-order vmcnt wait covers both and no load into registers is in
    // flight across the ring: the compiler's own wait for such a load, at
    // the ring's loop header, emptied the ring once every S chunks. Lane tid
    // fills 16 B at byte i * kBlock * 16 + tid * 16 of a stage: row
    // wrow + i * RPI, physical slot tid % LPR, which holds logical 16-B
    // column slot (tid % LPR) ^ sw(row), sw(row) = 2 * (row & 3); the four
    // rows one 16-lane transposed read addresses then fall in four distinct
    // 32-B bank groups without padding. The activation fragment f = ks * RBT + j
    // (K step ks, row block j) of a stage sits at S * SB + stage * SA + f * 1024,
    // in the gather's operand order (lane l's 16 B at l * 16).
    constexpr int OPS = NI + NA;  // vector memory instructions per lane per chunk
    static_assert((S - 1) * OPS < 64, "vmcnt is a 6-bit counter");
    static_assert(RPI % 4 == 0, "the rows a lane fills share their swizzle");
    static_assert(kLdsBytes <= 160 * 1024, "LDS");
    const int gcol_d = min(tile * HT + 8 * ((tid % LPR) ^ (2 * (wrow & 3))), h - 8);
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    // Every step issues the same instructions (a static vmcnt count, and no
    // branch for the compiler's own waits to merge): rows past the split
    // re-read its last row (zeroed in LDS once landed, below), chunks past its
    // last read that one row again (a few cache lines; never multiplied).
    auto issue = [&](int k, int s) {
      const bool live = k < nch;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int r = live ? min(k * kMcCK + wrow + i * RPI, cw - 1) : cw - 1;
        __builtin_amdgcn_global_load_lds(md + (size_t)(c0 + r) * (size_t)h + gcol_d,
                                         (lds_void*)(lds + s * SB + i * kBlock * 16 + wave * 1024), 16, 0, kMcNtAux);
      }
      const int q = c0 / kMcCK + min(k, nch - 1);
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int f = wv + 4 * i;
        const bool own = f < NFA;
        const int ks = own ? f / RBT : 0, j = own ? f % RBT : 0;
        const size_t frag = ((size_t)q * KS + ks) * (size_t)rbk_n + (size_t)min(j, rbk_n - 1);
        char* dst = own ? lds + S * SB + s * SA + f * 1024 : lds + S * (SB + SA);
        __builtin_amdgcn_global_load_lds(xg + frag * 512 + (size_t)lane * 8, (lds_void*)dst, 16, 0, 0);
      }
    };
    // The lane's transposed-read address (LDS bytes) of 16-column block nb,
    // stage 0, K step 0: row rr = 8 * lg + li / 4 (and rr + 4), logical
    // columns cb + 16 * nb + 4 * (li & 3) .. + 3.
    const int rr = 8 * lg + (li >> 2);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_char*)lds;
    uint32_t rd[NBK];
#pragma unroll
    for (int nb = 0; nb < NBK; ++nb) {
      const int lc = (cb + 16 * nb) / 8 + ((li & 3) >> 1);
      rd[nb] = lds0 + (uint32_t)(rr * RB + (lc ^ (2 * (rr & 3))) * 16 + (li & 1) * 8);
    }
    // The reads are inline asm: the compiler cannot tell the DMA stages
    // apart and would wait for every DMA in flight before each LDS read.
    // Their results are used only after the lgkmcnt wait (the empty asm
    // statements order each result after it).
    // The lane's activation-operand address (LDS bytes) of its row block, stage 0, K step 0.
    const uint32_t ra = lds0 + (uint32_t)(S * SB + (rb >> 4) * 1024 + lane * 16);
    auto compute_d = [&](int s) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        s4 lo[NBK], hi[NBK];
        s8 af[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) mc_read_b128(af[mb], ra + (uint32_t)(s * SA + (ks * RBT + mb) * 1024));
#pragma unroll
        for (int nb = 0; nb < NBK; ++nb) {
          const uint32_t ad = rd[nb] + (uint32_t)(s * SB + ks * 32 * RB);
          mc_read_tr_pair<4 * RB>(lo[nb], hi[nb], ad);
        }
        mc_lds_wait();
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) mc_after_wait8(af[mb]);
#pragma unroll
        for (int nb = 0; nb < NBK; ++nb) {
          mc_after_wait(lo[nb]);
          mc_after_wait(hi[nb]);
          const s8 bf = {lo[nb][0], lo[nb][1], lo[nb][2], lo[nb][3], hi[nb][0], hi[nb][1], hi[nb][2], hi[nb][3]};
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) acc[mb][nb] = mfma16x16x32<DT>(af[mb], bf, acc[mb][nb]);
        }
      }
    };
#pragma unroll
    for (int s = 0; s < S - 1; ++s) issue(s, s);
    for (int k0 = 0;; k0 += S) {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        if (k0 + s >= nch) goto mc_dma_done;
        // chunk k0 + s: this lane's loads have landed once at most the
        // S - 2 later chunks' are in flight; after the barrier every lane's
        // have, and every wave is done with the stage read last step.
        mc_wait_vm<(S - 2) * OPS>();
        __builtin_amdgcn_s_barrier();
        if ((k0 + s + 1) * kMcCK > cw) {
          // the split's ragged last chunk: its rows past cw hold row cw - 1
          const int z0 = cw - (k0 + s) * kMcCK;
#pragma unroll
          for (int i = 0; i < NI; ++i)
            if (wrow + i * RPI >= z0)
              *reinterpret_cast<u32x4*>(lds + s * SB + i * kBlock * 16 + tid * 16) = u32x4{0u, 0u, 0u, 0u};
          mc_lds_wait();
          __builtin_amdgcn_s_barrier();
        }
        issue(k0 + s + S - 1, (s + S - 1) % S);
        compute_d(s);
      }
    }
  mc_dma_done:
    mc_wait_vm<0>();  // no DMA into this workgroup's LDS outlives it
#endif
  } else {
  u32x4 wA[NI], wB[NI], aA[MB][KS], aB[MB][KS];
  load_w(wA, 0);
  load_a(aA, 0);
  load_w(wB, min(1, nch - 1));
  load_a(aB, min(1, nch - 1));

  auto store = [&](const u32x4 (&wr)[NI], int k, int buf) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const bool ok = k * kMcCK + wrow + i * RPI < cw;
      *reinterpret_cast<u32x4*>(&ws[buf][(wrow + i * RPI) * WSTR + wcol]) = ok ? wr[i] : u32x4{0u, 0u, 0u, 0u};
    }
  };

  auto compute = [&](const u32x4 (&af)[MB][KS], int buf) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int nb = 0; nb < NBK; ++nb) {
        // Lane t of group lg addresses row 32*ks + 8*lg + t/4 (then + 4),
        // columns n0 + 4*(t%4) .. +3; it receives column n0 + t of the
        // group's rows.
        const T* p = &ws[buf][(32 * ks + 8 * lg + (li >> 2)) * WSTR + cb + 16 * nb + 4 * (li & 3)];
        const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)p);
        const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p + 4 * WSTR));
        const s8 bf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          acc[mb][nb] = mfma16x16x32<DT>(__builtin_bit_cast(s8, af[mb][ks]), bf, acc[mb][nb]);
      }
  };

  // Buffer b holds chunk k (k % 2 == b); the barrier after each store also
  // orders the previous reads of the other buffer before its next store.
  // Loads past the split's last chunk re-read it (never used).
  for (int k = 0; k < nch; k += 2) {
    store(wA, k, 0);
    __syncthreads();
    u32x4 a0[MB][KS];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) a0[mb][ks] = aA[mb][ks];
    load_w(wA, min(k + 2, nch - 1));
    load_a(aA, min(k + 2, nch - 1));
    compute(a0, 0);
    if (k + 1 < nch) {
      store(wB, k + 1, 1);
      __syncthreads();
      u32x4 a1[MB][KS];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) a1[mb][ks] = aB[mb][ks];
      load_w(wB, min(k + 3, nch - 1));
      load_a(aB, min(k + 3, nch - 1));
      compute(a1, 1);
    }
  }
  }

  // acc[mb][nb][j]: batch row rb + 16*mb + 4*lg + j, output column
  // tile*HT + cb + 16*nb + li.
  const int rcol = tile * HT + cb + li;
  if (a.splits > 1) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int b = rb + 16 * mb + 4 * lg + j;
          const int r = rcol + 16 * nb;
          if (b < a.batch && r < h)
            __hip_atomic_store(a.partial + ((size_t)split * (size_t)a.batch + (size_t)b) * (size_t)h + r,
                               acc[mb][nb][j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // also: every wave's staging reads and DMAs are done, so is_last may take the first word
    if (tid == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(&a.tickets[tile], 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      is_last = (prev == (uint32_t)(a.splits - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (!is_last) return;
    // Every split's partials of the lane's outputs, GS splits per round trip,
    // summed in split order (clamped addresses for outputs that are unused).
    // At most 32 loads in flight per lane: more raised the register count of
    // the 64 x 128 tile to one wave per SIMD and slowed it down. A split's
    // base is uniform; the lane keeps 32-bit offsets (batch * h < 2^31,
    // checked by the plan).
    constexpr int NOUT = MB * NBK * 4;
    constexpr int GS = NOUT >= 32 ? 1 : (32 / NOUT >= 8 ? 8 : 32 / NOUT);
    const size_t step = (size_t)a.batch * (size_t)h;
    int roff[MB][4], coff[NBK];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j) roff[mb][j] = min(rb + 16 * mb + 4 * lg + j, a.batch - 1) * h;
#pragma unroll
    for (int nb = 0; nb < NBK; ++nb) coff[nb] = min(rcol + 16 * nb, h - 1);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[mb][nb][j] = 0.0f;
    int sp = 0;
    for (; sp + GS <= a.splits; sp += GS) {
      float t[MB][NBK][4][GS];
#pragma unroll
      for (int i = 0; i < GS; ++i) {
        const float* ps = a.partial + (size_t)(sp + i) * step;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              t[mb][nb][j][i] = __hip_atomic_load(ps + (roff[mb][j] + coff[nb]), __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < GS; ++i) acc[mb][nb][j] += t[mb][nb][j][i];
    }
    for (; sp < a.splits; ++sp) {
      float t[MB][NBK][4];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            t[mb][nb][j] = __hip_atomic_load(a.partial + (size_t)sp * step + (roff[mb][j] + coff[nb]),
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[mb][nb][j] += t[mb][nb][j];
    }
  }

  T* __restrict__ out = static_cast<T*>(a.out);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int b = rb + 16 * mb + 4 * lg + j;
        const int r = rcol + 16 * nb;
        if (b < a.batch && r < h) out[(long long)b * a.out_row_stride + r] = E::from_f32(acc[mb][nb][j]);
      }
  if (a.splits > 1 && tid == 0) {
    __hip_atomic_store(&a.tickets[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int DT, int BT, int HT, bool DMA>
__global__ __launch_bounds__(kBlock) void nm_spmm_mc_kernel(SpmmArgs a) {
  mc_tile<DT, BT, HT, DMA>(a, (int)blockIdx.x);
}

// Several products of the same activations in one grid (sibling Linears:
// q/k/v, gate/up): product i owns workgroups first[i] .. first[i + 1] - 1,
// with its own weights, gathered activations, outputs, partials and
// arrival counters, the same tile width, batch and split count.
constexpr int kMcMaxGroup = NM_MC_MAX_GROUP;
struct McGroupArgs {
  SpmmArgs p[kMcMaxGroup];
  int first[kMcMaxGroup];
  int n;
};

template <int DT, int BT, int HT, bool DMA>
__global__ __launch_bounds__(kBlock) void nm_spmm_mc_group_kernel(McGroupArgs g) {
  const int b = (int)blockIdx.x;
  int i = 0;
#pragma unroll
  for (int j = 1; j < kMcMaxGroup; ++j) i += (j < g.n && b >= g.first[j]) ? 1 : 0;
  mc_tile<DT, BT, HT, DMA>(g.p[i], b - g.first[i]);
}

// The gathered activations xg[b, c] = x[b, (c/nnz)*m + mat_index[c]] for
// c < w, zero for positions outside x, for w <= c < wp and for rows past the
// batch. Lane i writes 8 consecutive columns of one row as one 16-B store:
// row-major (FRAG = false: rows wp apart, wp a multiple of 8; `batch` rows)
// or in the matrix-core kernel's operand order (FRAG = true: lane i fills
// 16-B slot i of the fragments described at nm_spmm_mc_kernel's load_a; wp
// a multiple of 64; rbk row blocks of 16 rows).
// SDT >= 0 (an element type): the activations are round_SDT(silu(x) * x2)
// of two inputs with the same row stride, computed in fp32 as the gate/up
// pair's epilogue does, only at the gathered positions.
template <bool FRAG, int SDT = -1>
__device__ __forceinline__ void gather_slot(const uint16_t* __restrict__ x, long long x_row_stride, int batch,
                                            const uint8_t* __restrict__ mat_index, int w, int wp, int nnz, int m,
                                            int K, int rbk, uint16_t* __restrict__ xg,
                                            const uint16_t* __restrict__ x2 = nullptr) {
  const int per_row = wp / 8;  // rows * per_row < 2^31 (host)
  const int i = (int)blockIdx.x * kBlock + (int)threadIdx.x;
  if (i >= (FRAG ? 16 * rbk : batch) * per_row) return;
  int b, c0;
  if (FRAG) {  // slot i: fragment i / 64 = (chunk * 2 + ks) * rbk + j, lane l = i % 64
    const int f = i >> 6, l = i & 63;
    const int j = f % rbk, qk = f / rbk;
    b = 16 * j + (l & 15);
    c0 = 32 * qk + 8 * (l >> 4);
  } else {
    b = i / per_row;
    c0 = (i - b * per_row) * 8;
  }
  const bool row_ok = b < batch;
  const uint16_t* __restrict__ xr = x + (long long)(row_ok ? b : 0) * x_row_stride;
  uint16_t v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int c = c0 + e;
    const int cc = c < w ? c : w - 1;  // clamped: the load stays in range
    const int p = (cc / nnz) * m + (int)mat_index[cc];
    uint16_t t = xr[p < K ? p : 0];
    if constexpr (SDT >= 0) {
      using E = Elem<SDT>;
      const uint16_t u = x2[(long long)(row_ok ? b : 0) * x_row_stride + (p < K ? p : 0)];
      t = E::from_f32(silu(E::to_f32(t)) * E::to_f32(u));
    }
    v[e] = (row_ok && c < w && p < K) ? t : (uint16_t)0;
  }
  u32x4 word;
  word.x = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
  word.y = (uint32_t)v[2] | ((uint32_t)v[3] << 16);
  word.z = (uint32_t)v[4] | ((uint32_t)v[5] << 16);
  word.w = (uint32_t)v[6] | ((uint32_t)v[7] << 16);
  *reinterpret_cast<u32x4*>(xg + (FRAG ? (long long)i * 8 : (long long)b * wp + c0)) = word;
}

template <bool FRAG>
__global__ __launch_bounds__(kBlock) void nm_gather_mc_kernel(const uint16_t* __restrict__ x, long long x_row_stride,
                                                            int batch, const uint8_t* __restrict__ mat_index, int w,
                                                            int wp, int nnz, int m, int K, int rbk,
                                                            uint16_t* __restrict__ xg) {
  gather_slot<FRAG>(x, x_row_stride, batch, mat_index, w, wp, nnz, m, K, rbk, xg);
}

// The operand-order gather of round_SDT(silu(gate) * up).
template <int SDT>
__global__ __launch_bounds__(kBlock) void nm_gather_mc_silu_kernel(const uint16_t* __restrict__ gate,
                                                                 const uint16_t* __restrict__ up,
                                                                 long long x_row_stride, int batch,
                                                                 const uint8_t* __restrict__ mat_index, int w,
                                                                 int wp, int nnz, int m, int K, int rbk,
                                                                 uint16_t* __restrict__ xg) {
  gather_slot<true, SDT>(gate, x_row_stride, batch, mat_index, w, wp, nnz, m, K, rbk, xg, up);
}

// The operand-order gathers of a group's products, product blockIdx.y each.
struct McGatherGroup {
  const uint8_t* mat_index[kMcMaxGroup];
  uint16_t* xg[kMcMaxGroup];
};

__global__ __launch_bounds__(kBlock) void nm_gather_mc_group_kernel(const uint16_t* __restrict__ x,
                                                                  long long x_row_stride, int batch, int w, int wp,
                                                                  int nnz, int m, int K, int rbk, McGatherGroup gg) {
  const int i = (int)blockIdx.y;
  gather_slot<true>(x, x_row_stride, batch, gg.mat_index[i], w, wp, nnz, m, K, rbk, gg.xg[i]);
}

typedef void (*McFn)(SpmmArgs);
typedef void (*McGroupFn)(McGroupArgs);

// fn[config: HT = 64, 128, 256][batch tile: 16, 32, 64, 128 rows]
// (no 128-row tile of 256 columns: its accumulators and operands exceed the
// register file; the plan does not take HT = 256 past 64 rows)
#define NM_MC_ROW(DT, HT, DMA)                                                                               \
  {&nm_spmm_mc_kernel<DT, 16, HT, DMA>, &nm_spmm_mc_kernel<DT, 32, HT, DMA>, &nm_spmm_mc_kernel<DT, 64, HT, DMA>, \
   &nm_spmm_mc_kernel<DT, 128, HT, DMA>}
#define NM_MC_ROW3(DT, HT, DMA)                                                                              \
  {&nm_spmm_mc_kernel<DT, 16, HT, DMA>, &nm_spmm_mc_kernel<DT, 32, HT, DMA>, &nm_spmm_mc_kernel<DT, 64, HT, DMA>, \
   nullptr}
#define NM_MC_TABLE(DT)                                                                                     \
  {NM_MC_ROW(DT, 64, false), NM_MC_ROW(DT, 128, false), NM_MC_ROW3(DT, 256, false), NM_MC_ROW(DT, 64, true), \
   NM_MC_ROW(DT, 128, true), NM_MC_ROW3(DT, 256, true)}
const McFn kMcKernelsF16[kMcNumConfigs][4] = NM_MC_TABLE(NM_DTYPE_F16);
const McFn kMcKernelsBF16[kMcNumConfigs][4] = NM_MC_TABLE(NM_DTYPE_BF16);
#undef NM_MC_ROW
#undef NM_MC_ROW3
#define NM_MC_ROW(DT, HT, DMA)                                                                     \
  {&nm_spmm_mc_group_kernel<DT, 16, HT, DMA>, &nm_spmm_mc_group_kernel<DT, 32, HT, DMA>,          \
   &nm_spmm_mc_group_kernel<DT, 64, HT, DMA>, &nm_spmm_mc_group_kernel<DT, 128, HT, DMA>}
#define NM_MC_ROW3(DT, HT, DMA)                                                                    \
  {&nm_spmm_mc_group_kernel<DT, 16, HT, DMA>, &nm_spmm_mc_group_kernel<DT, 32, HT, DMA>,          \
   &nm_spmm_mc_group_kernel<DT, 64, HT, DMA>, nullptr}
const McGroupFn kMcGroupKernelsF16[kMcNumConfigs][4] = NM_MC_TABLE(NM_DTYPE_F16);
const McGroupFn kMcGroupKernelsBF16[kMcNumConfigs][4] = NM_MC_TABLE(NM_DTYPE_BF16);
#undef NM_MC_TABLE
#undef NM_MC_ROW
#undef NM_MC_ROW3

constexpr int kMcTileCols[kMcNumConfigs] = {64, 128, 256, 64, 128, 256};
constexpr int kMcCUs = 256;  // MI355X compute units; split counts aim at about this many workgroups

inline int ceil_div_mc(int a, int b) { return (a + b - 1) / b; }

struct McPlan {
  int cfg, splits, rows, tiles, blocks, wp;
  size_t xg_off, xg_bytes, workspace;
};

// Plan, fitted to graph-replay sweeps of the DMA configurations x 1-8 splits
// at the Llama-3.1-8B, Qwen3-14B and Qwen3-32B shapes, 16 / 32 / 64 rows (and the
// Llama-3.1-8B shapes at 96 / 128 rows).
// Up to 1024 outputs: register-staged 64-column tiles, about one workgroup
// per CU (256 / tiles splits, at most 8). Otherwise the DMA-staged tile width
// and split count are chosen together: the grid of the most workgroups that
// still runs in one round (at most one per CU; a second round of a few
// workgroups costs more than it brings), ties broken by
//  * splits of at most 2560 compressed rows (deep K runs slower per split);
//  * up to 16 rows: 64-column tiles, then 128, then 256;
//  * past 16 rows: fewer splits (their partials, [splits, batch, h] fp32,
//    grow with the rows), then 128-, 64-, 256-column tiles;
//  * past 32 rows, among grids that fit one round: splits of at most 2560
//    compressed rows, then 64-column tiles, then the most workgroups (the
//    grouped Llama-3.1-8B q/k/v on 64-column tiles and 192 workgroups ran 17-19%
//    faster than on 128-column tiles and 240 at 40-64 rows, and the 64-column
//    tiles were faster at every Llama-3.1-8B product at 96-128 rows; Qwen3
//    down's deeper 64-column splits were 3-8% slower); no 256-column tile past
//    64 rows;
// and from 33 to 64 rows a plan whose partials would reach a quarter of the
// weight bytes gives way to the widest grid without splits, when that has at
// least half its workgroups. Each split is whole chunks of 64 columns. Workspace:
// arrival counters, the partials [splits, batch, h] fp32 when splits > 1,
// then the gathered activations in operand order (ceil(batch / 16) blocks of
// 16 rows x wp columns, wp = w rounded up to whole chunks).
// A group (n products of the same activations, output widths hs[0 .. n-1])
// is planned as one product whose tiles are all the products' tiles: one
// tile width and split count; partials and gathered activations per product,
// one after another.
int make_mc_plan(int batch, int n, const int* hs, int w, int nnz, int m, int cfg, int splits, McPlan* p) {
  if (batch < 1 || batch > NM_MC_MAX_BATCH || n < 1 || n > kMcMaxGroup || !hs) return NM_ERR_BAD_SHAPE;
  if (w <= 0 || nnz <= 0 || m <= 0 || m > 256 || nnz > m) return NM_ERR_BAD_SHAPE;
  long long hsum = 0;
  int hmax = 0;
  for (int i = 0; i < n; ++i) {
    if (hs[i] <= 0) return NM_ERR_BAD_SHAPE;
    if (hs[i] % 128 != 0) return NM_ERR_H_NOT_MULTIPLE_128;
    hsum += hs[i];
    hmax = hs[i] > hmax ? hs[i] : hmax;
  }
  if (w % nnz != 0) return NM_ERR_W_NOT_MULTIPLE_NNZ;
  if ((long long)(w / nnz) * (long long)m > 0x7fffffffLL || w > 0x7fffffff - kMcCK) return NM_ERR_BAD_SHAPE;
  if ((long long)batch * (long long)(w / 8 + kMcCK) > 0x7fffffffLL) return NM_ERR_BAD_SHAPE;
  if ((long long)batch * (long long)hmax > 0x7fffffffLL) return NM_ERR_BAD_SHAPE;  // the reduction's 32-bit offsets
  if (cfg >= kMcNumConfigs) return NM_ERR_BAD_CONFIG;
  if (batch > 64 && kMcTileCols[cfg < 0 ? 0 : cfg] == 256) return NM_ERR_BAD_CONFIG;  // no 128 x 256 tile
  const int wp = ceil_div_mc(w, kMcCK) * kMcCK;
  auto tiles_of = [&](int c) {
    int t = 0;
    for (int i = 0; i < n; ++i) t += ceil_div_mc(hs[i], kMcTileCols[c]);
    return t;
  };
  // (tiles, splits, rows per split) of a configuration and a requested split count
  auto shape_of = [&](int c, int sp, int* tiles_out, int* rows_out) {
    if (sp > wp / kMcCK) sp = wp / kMcCK;
    const int r = ceil_div_mc(ceil_div_mc(w, sp), kMcCK) * kMcCK;
    *tiles_out = tiles_of(c);
    *rows_out = r;
    return ceil_div_mc(w, r);
  };
  if (cfg < 0 && hmax <= 1024) cfg = 0;
  if (cfg >= 0 && cfg < 3 && splits <= 0) {  // register-staged: about one workgroup per CU
    const int t = tiles_of(cfg);
    splits = (kMcCUs + t / 2) / t;
    splits = splits < 1 ? 1 : (splits > 8 ? 8 : splits);
  } else if (cfg < 0 || splits <= 0) {
    // search the DMA configurations (or the given one) x split counts (or the given one)
    const int c_lo = cfg < 0 ? 3 : cfg, c_hi = cfg < 0 ? 5 : cfg;
    const int s_lo = splits > 0 ? splits : 1, s_hi = splits > 0 ? splits : 8;
    const int pref_small[3] = {0, 1, 2};  // ranks of HT = 64, 128, 256 up to 16 rows (lower is better)
    const int pref_large[3] = {1, 0, 2};  // 17-64 rows
    int best_c = -1, best_s = 0, best_b = 0, best_r = 0, free_c = -1, free_b = 0;
    auto better = [&](int c, int sp, int b, int r) {
      if (best_c < 0) return true;
      const bool fits = b <= kMcCUs, best_fits = best_b <= kMcCUs;
      if (fits != best_fits) return fits;
      if (!fits) return b < best_b;  // nothing fits one round: the smallest grid
      const bool deep = r > 2560, best_deep = best_r > 2560;
      if (batch > 32) {  // past 32 rows: shallow splits, then 64-column tiles, then the most workgroups
        if (deep != best_deep) return !deep;
        if ((kMcTileCols[c] == 64) != (kMcTileCols[best_c] == 64)) return kMcTileCols[c] == 64;
      }
      if (b != best_b) return b > best_b;
      if (deep != best_deep) return !deep;
      if (batch > 16 && sp != best_s) return sp < best_s;
      const int* pref = batch > 16 ? pref_large : pref_small;
      return pref[c - 3] < pref[best_c - 3];
    };
    for (int c = c_lo; c <= c_hi; ++c)
      for (int sp = s_lo; sp <= s_hi; ++sp) {
        if (batch > 64 && kMcTileCols[c] == 256) continue;
        int t, r;
        const int se = shape_of(c, sp, &t, &r);
        if (se != sp && splits <= 0) continue;  // the same grid as a smaller request
        const long long b = (long long)t * se;
        if (b > 0x7fffffffLL) continue;
        if (better(c, se, (int)b, r)) {
          best_c = c, best_s = se, best_b = (int)b, best_r = r;
        }
        if (se == 1 && b <= kMcCUs && b > free_b) free_c = c, free_b = (int)b;
      }
    if (best_c < 0) return NM_ERR_BAD_SHAPE;
    const long long part4 = 4LL * best_s * batch;  // partials written and read, relative to 2 * w weight bytes
    if (batch > 32 && batch <= 64 && splits <= 0 && best_s > 1 && part4 * 4 >= (long long)w && free_c >= 0 &&
        2 * free_b >= best_b) {
      best_c = free_c;
      best_s = 1;
    }
    cfg = best_c;
    splits = best_s;
  }
  int tiles, rows;
  splits = shape_of(cfg, splits, &tiles, &rows);
  if (tiles > kMaxTickets || (long long)tiles * splits > 0x7fffffffLL) return NM_ERR_BAD_SHAPE;
  p->cfg = cfg;
  p->splits = splits;
  p->rows = rows;
  p->tiles = tiles;
  p->blocks = tiles * splits;
  p->wp = wp;
  const size_t part = splits > 1 ? (size_t)splits * (size_t)batch * (size_t)hsum * sizeof(float) : (size_t)0;
  p->xg_off = ((size_t)NM_TICKET_BYTES + part + 255) / 256 * 256;
  p->xg_bytes = (size_t)ceil_div_mc(batch, 16) * 16 * (size_t)wp * 2;  // per product, a multiple of 2 KB
  p->workspace = p->xg_off + (size_t)n * p->xg_bytes;
  return NM_OK;
}

int make_mc_plan(int batch, int h, int w, int nnz, int m, int cfg, int splits, McPlan* p) {
  return make_mc_plan(batch, 1, &h, w, nnz, m, cfg, splits, p);
}

// nm_spmm_mc, and with x2 (the up projection's output, rows x_row_stride
// apart like x) nm_spmm_mc_silu_mul: the gather then forms round_T(silu(x)
// * x2) at the gathered positions.
int spmm_mc_run(int dtype, const void* x, const void* x2, long long x_row_stride, int batch, const void* mat_data,
                const uint8_t* mat_index, void* out, long long out_row_stride, void* workspace,
                size_t workspace_bytes, int h, int w, int nnz, int m, int config_id, int splits, void* stream) {
  if (dtype != NM_DTYPE_F16 && dtype != NM_DTYPE_BF16) return NM_ERR_BAD_CONFIG;
  McPlan p;
  const int rc = make_mc_plan(batch, h, w, nnz, m, config_id, splits, &p);
  if (rc != NM_OK) return rc;
  if (!x || !mat_data || !mat_index || !out || !workspace) return NM_ERR_NULL_POINTER;
  const long long K = (long long)(w / nnz) * (long long)m;
  if (x_row_stride < K || out_row_stride < h) return NM_ERR_BAD_SHAPE;
  if (((uintptr_t)mat_data & 15u) != 0 || ((uintptr_t)workspace & 255u) != 0) return NM_ERR_MISALIGNED;
  if (workspace_bytes < p.workspace) return NM_ERR_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  void* xg = static_cast<char*>(workspace) + p.xg_off;
  const int rbk = ceil_div_mc(batch, 16);  // row blocks of 16 stored (operand order, zero rows past the batch)
  const long long gathered = (long long)16 * rbk * (long long)(p.wp / 8);
  const unsigned gblocks = (unsigned)((gathered + kBlock - 1) / kBlock);
  if (!x2)
    hipLaunchKernelGGL(nm_gather_mc_kernel<true>, dim3(gblocks), dim3(kBlock), 0, st,
                       static_cast<const uint16_t*>(x), x_row_stride, batch, mat_index, w, p.wp, nnz, m, (int)K,
                       rbk, static_cast<uint16_t*>(xg));  // fp16 and bf16 alike: a copy of 16-bit words
  else
    hipLaunchKernelGGL(dtype == NM_DTYPE_F16 ? nm_gather_mc_silu_kernel<NM_DTYPE_F16>
                                             : nm_gather_mc_silu_kernel<NM_DTYPE_BF16>,
                       dim3(gblocks), dim3(kBlock), 0, st, static_cast<const uint16_t*>(x),
                       static_cast<const uint16_t*>(x2), x_row_stride, batch, mat_index, w, p.wp, nnz, m, (int)K,
                       rbk, static_cast<uint16_t*>(xg));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  SpmmArgs a;
  memset(&a, 0, sizeof(a));
  a.x = xg;
  a.x_row_stride = rbk;  // operand-order activations: the row blocks stored
  a.mat_data = mat_data;
  a.mat_index = mat_index;
  a.out = out;
  a.out_row_stride = out_row_stride;
  a.tickets = static_cast<uint32_t*>(workspace);
  a.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + NM_TICKET_BYTES);
  a.batch = batch;
  a.h = h;
  a.tiles = p.tiles;
  a.w = w;
  a.nnz = nnz;
  a.m = m;
  a.K = (int)K;
  a.splits = p.splits;
  a.rows_per_split = p.rows;
  const int bt = batch <= 16 ? 0 : (batch <= 32 ? 1 : (batch <= 64 ? 2 : 3));
  const McFn fn = (dtype == NM_DTYPE_F16 ? kMcKernelsF16 : kMcKernelsBF16)[p.cfg][bt];
  hipLaunchKernelGGL(fn, dim3(p.blocks), dim3(kBlock), 0, st, a);
  e = hipGetLastError();
  return e == hipSuccess ? NM_OK : (int)e;
}

}  // namespace
}  // namespace nm_hip

using namespace nm_hip;

extern "C" {

size_t nm_spmm_mc_workspace_bytes(int batch, int h, int w, int nnz, int m, int config_id, int splits) {
  McPlan p;
  return make_mc_plan(batch, h, w, nnz, m, config_id, splits, &p) == NM_OK ? p.workspace : 0;
}

int nm_spmm_mc_plan(int batch, int h, int w, int nnz, int m, int config_id, int splits, int* out_config_id,
                    int* out_splits, int* out_blocks, int* out_rows_per_block) {
  McPlan p;
  const int rc = make_mc_plan(batch, h, w, nnz, m, config_id, splits, &p);
  if (rc != NM_OK) return rc;
  if (out_config_id) *out_config_id = p.cfg;
  if (out_splits) *out_splits = p.splits;
  if (out_blocks) *out_blocks = p.blocks;
  if (out_rows_per_block) *out_rows_per_block = p.rows;
  return NM_OK;
}

int nm_gather_columns(int dtype, const void* x, long long x_row_stride, int rows, const uint8_t* mat_index, int w,
                      int nnz, int m, void* out, long long out_row_stride, void* stream) {
  if (dtype != NM_DTYPE_F16 && dtype != NM_DTYPE_BF16) return NM_ERR_BAD_CONFIG;
  if (rows < 1 || w <= 0 || nnz <= 0 || m <= 0 || m > 256 || nnz > m || w % nnz != 0) return NM_ERR_BAD_SHAPE;
  if (!x || !mat_index || !out) return NM_ERR_NULL_POINTER;
  const long long K = (long long)(w / nnz) * (long long)m;
  const long long wp = ((long long)w + 7) / 8 * 8;
  if (K > 0x7fffffffLL || x_row_stride < K || out_row_stride < wp || out_row_stride % 8 != 0 ||
      out_row_stride > 0x7fffffffLL || (long long)rows * (out_row_stride / 8) > 0x7fffffffLL)
    return NM_ERR_BAD_SHAPE;
  if (((uintptr_t)out & 15u) != 0) return NM_ERR_MISALIGNED;
  // rows of out_row_stride elements: every column past w is written as zero
  const long long lanes = (long long)rows * (out_row_stride / 8);
  hipLaunchKernelGGL(nm_gather_mc_kernel<false>, dim3((unsigned)((lanes + kBlock - 1) / kBlock)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), x_row_stride, rows,
                     mat_index, w, (int)out_row_stride, nnz, m, (int)K, 0, static_cast<uint16_t*>(out));
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? NM_OK : (int)e;
}

int nm_spmm_mc(int dtype, const void* x, long long x_row_stride, int batch, const void* mat_data,
               const uint8_t* mat_index, void* out, long long out_row_stride, void* workspace, size_t workspace_bytes,
               int h, int w, int nnz, int m, int config_id, int splits, void* stream) {
  return spmm_mc_run(dtype, x, nullptr, x_row_stride, batch, mat_data, mat_index, out, out_row_stride, workspace,
                     workspace_bytes, h, w, nnz, m, config_id, splits, stream);
}

int nm_spmm_mc_silu_mul(int dtype, const void* gate, const void* up, long long x_row_stride, int batch,
                        const void* mat_data, const uint8_t* mat_index, void* out, long long out_row_stride,
                        void* workspace, size_t workspace_bytes, int h, int w, int nnz, int m, int config_id,
                        int splits, void* stream) {
  if (!up) return NM_ERR_NULL_POINTER;
  return spmm_mc_run(dtype, gate, up, x_row_stride, batch, mat_data, mat_index, out, out_row_stride, workspace,
                     workspace_bytes, h, w, nnz, m, config_id, splits, stream);
}

size_t nm_spmm_mc_group_workspace_bytes(int batch, int n, const int* h, int w, int nnz, int m, int config_id,
                                        int splits) {
  McPlan p;
  return make_mc_plan(batch, n, h, w, nnz, m, config_id, splits, &p) == NM_OK ? p.workspace : 0;
}

int nm_spmm_mc_group_plan(int batch, int n, const int* h, int w, int nnz, int m, int config_id, int splits,
                          int* out_config_id, int* out_splits, int* out_blocks, int* out_rows_per_block) {
  McPlan p;
  const int rc = make_mc_plan(batch, n, h, w, nnz, m, config_id, splits, &p);
  if (rc != NM_OK) return rc;
  if (out_config_id) *out_config_id = p.cfg;
  if (out_splits) *out_splits = p.splits;
  if (out_blocks) *out_blocks = p.blocks;
  if (out_rows_per_block) *out_rows_per_block = p.rows;
  return NM_OK;
}

int nm_spmm_mc_group(int dtype, const void* x, long long x_row_stride, int batch, int n, const void* const* mat_data,
                     const uint8_t* const* mat_index, void* const* out, const long long* out_row_stride,
                     const int* h, void* workspace, size_t workspace_bytes, int w, int nnz, int m, int config_id,
                     int splits, void* stream) {
  if (dtype != NM_DTYPE_F16 && dtype != NM_DTYPE_BF16) return NM_ERR_BAD_CONFIG;
  if (!mat_data || !mat_index || !out || !out_row_stride || !h) return NM_ERR_NULL_POINTER;
  McPlan p;
  const int rc = make_mc_plan(batch, n, h, w, nnz, m, config_id, splits, &p);
  if (rc != NM_OK) return rc;
  if (!x || !workspace) return NM_ERR_NULL_POINTER;
  const long long K = (long long)(w / nnz) * (long long)m;
  if (x_row_stride < K) return NM_ERR_BAD_SHAPE;
  for (int i = 0; i < n; ++i) {
    if (!mat_data[i] || !mat_index[i] || !out[i]) return NM_ERR_NULL_POINTER;
    if (out_row_stride[i] < h[i]) return NM_ERR_BAD_SHAPE;
    if (((uintptr_t)mat_data[i] & 15u) != 0) return NM_ERR_MISALIGNED;
  }
  if (((uintptr_t)workspace & 255u) != 0) return NM_ERR_MISALIGNED;
  if (workspace_bytes < p.workspace) return NM_ERR_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int rbk = ceil_div_mc(batch, 16);
  McGatherGroup gg;
  memset(&gg, 0, sizeof(gg));
  McGroupArgs g;
  memset(&g, 0, sizeof(g));
  g.n = n;
  size_t part_off = 0;
  int tile_off = 0, block_off = 0;
  for (int i = 0; i < n; ++i) {
    uint16_t* xg = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + p.xg_off + (size_t)i * p.xg_bytes);
    gg.mat_index[i] = mat_index[i];
    gg.xg[i] = xg;
    SpmmArgs& a = g.p[i];
    const int tiles = ceil_div_mc(h[i], kMcTileCols[p.cfg]);
    a.x = xg;
    a.x_row_stride = rbk;  // operand-order activations: the row blocks stored
    a.mat_data = mat_data[i];
    a.mat_index = mat_index[i];
    a.out = out[i];
    a.out_row_stride = out_row_stride[i];
    a.tickets = static_cast<uint32_t*>(workspace) + tile_off;
    a.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + NM_TICKET_BYTES) + part_off;
    a.batch = batch;
    a.h = h[i];
    a.tiles = tiles;
    a.w = w;
    a.nnz = nnz;
    a.m = m;
    a.K = (int)K;
    a.splits = p.splits;
    a.rows_per_split = p.rows;
    g.first[i] = block_off;
    tile_off += tiles;
    block_off += tiles * p.splits;
    part_off += p.splits > 1 ? (size_t)p.splits * (size_t)batch * (size_t)h[i] : (size_t)0;
  }
  const long long gathered = (long long)16 * rbk * (long long)(p.wp / 8);
  const unsigned gblocks = (unsigned)((gathered + kBlock - 1) / kBlock);
  hipLaunchKernelGGL(nm_gather_mc_group_kernel, dim3(gblocks, (unsigned)n), dim3(kBlock), 0, st,
                     static_cast<const uint16_t*>(x), x_row_stride, batch, w, p.wp, nnz, m, (int)K, rbk, gg);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  const int bt = batch <= 16 ? 0 : (batch <= 32 ? 1 : (batch <= 64 ? 2 : 3));
  const McGroupFn fn = (dtype == NM_DTYPE_F16 ? kMcGroupKernelsF16 : kMcGroupKernelsBF16)[p.cfg][bt];
  hipLaunchKernelGGL(fn, dim3(p.blocks), dim3(kBlock), 0, st, g);
  e = hipGetLastError();
  return e == hipSuccess ? NM_OK : (int)e;
}

}  // extern "C"
