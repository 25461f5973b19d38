/*
 * nm_gemv_ref.c — CPU oracle for the shared-mask N:M sparse GEMV.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or the timed CPU baseline), never on the product path.
 *
 * Restates, in plain C, the arithmetic of the reference kernels
 * (triton_spmv.py:56-115 and triton_spmv.py:149-214):
 *
 *   out_f32[r] = sum over g ascending, then i ascending (triton_spmv.py:175-207)
 *                of fmaf(f32(mat_data[g*N+i, r]), f32(vec[(g*M + mat_index[g,i]) * stride]), acc)
 *
 * with fp32 fused multiply-add (the inline PTX fma.rn.f32 of
 * triton_spmv.py:24-35) and a round-to-nearest-even cast of the fp32 result
 * to the input type (`out_fp32.to(vec.dtype)`, triton_spmv.py:318). This is
 * the reference's in-program order with a single program spanning all groups;
 * its split-K atomics (triton_spmv.py:209-214) only reorder the same sum.
 *
 * Conversions are written from the IEEE-754 binary16 / bfloat16 definitions
 * (no hardware conversion instructions) so the oracle does not share an
 * implementation with the GPU path. A position g*M + mat_index[g,i] >= K
 * contributes zero, matching the library's documented behaviour for
 * out-of-range positions (the reference reads outside vec there).
 *
 * Pinned by tests/test_oracle.py: the conversions exhaustively against
 * numpy's IEEE conversions; the GEMV against closed forms (one-hot KATs,
 * zero vectors, linearity under powers of two) and against an fp64 dense
 * matvec on the scattered weight.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static inline uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* binary16 -> binary32, exact. */
float nm_oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0x1fu) return bits_f32(sign | 0x7f800000u | (man << 13)); /* inf / nan */
  if (exp == 0) {
    if (man == 0) return bits_f32(sign);                                 /* +-0 */
    /* subnormal: man * 2^-24 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* binary32 -> binary16, round to nearest, ties to even; overflow -> inf. */
uint16_t nm_oracle_f32_to_f16(float f) {
  const uint32_t u = f32_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t exp = (u >> 23) & 0xffu;
  const uint32_t man = u & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
  const int e = (int)exp - 127; /* unbiased */
  if (e > 15) return (uint16_t)(sign | 0x7c00u);
  if (e >= -14) {
    /* normal range: keep 10 bits, round the dropped 13 bits */
    uint32_t half = ((uint32_t)(e + 15) << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half += 1u; /* may carry into exp: ok */
    return (uint16_t)(sign | half);
  }
  if (e < -25) return sign; /* below half of the smallest subnormal */
  /* subnormal: value = (1.man) * 2^e, target unit 2^-24 */
  const uint32_t full = man | 0x800000u;         /* 24-bit significand, value full * 2^(e-23) */
  const int shift = -e - 1;                       /* full * 2^(e-23) / 2^-24 = full >> (-e - 1) */
  uint32_t q = full >> shift;
  const uint32_t rem = full & ((1u << shift) - 1u);
  const uint32_t halfway = 1u << (shift - 1);
  if (rem > halfway || (rem == halfway && (q & 1u))) q += 1u;
  return (uint16_t)(sign | q);
}

float nm_oracle_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* binary32 -> bfloat16, round to nearest, ties to even; NaN -> 0x7fc0. */
uint16_t nm_oracle_f32_to_bf16(float f) {
  const uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  const uint32_t lower = u & 0xffffu;
  uint32_t upper = u >> 16;
  if (lower > 0x8000u || (lower == 0x8000u && (upper & 1u))) upper += 1u;
  return (uint16_t)upper;
}

enum { NM_OR_F16 = 0, NM_OR_BF16 = 1, NM_OR_F32 = 2 };

static inline float load_elem(const void* p, size_t i, int dtype) {
  if (dtype == NM_OR_F16) return nm_oracle_f16_to_f32(((const uint16_t*)p)[i]);
  if (dtype == NM_OR_BF16) return nm_oracle_bf16_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

/*
 * The GEMV. vec has K = (w / nnz) * m elements at stride vec_stride;
 * mat_data is [w, h] row-major; mat_index is [w/nnz, nnz]. Writes the fp32
 * accumulators to out_f32 (h floats, required) and the rounded result to out
 * (same element type as the inputs; may be NULL). Returns 0, or -1 on bad
 * arguments.
 */
int nm_oracle_gemv(int dtype, const void* vec, long long vec_stride, const void* mat_data,
                   const uint8_t* mat_index, float* out_f32, void* out, int h, int w, int nnz,
                   int m) {
  if (h <= 0 || w <= 0 || nnz <= 0 || m <= 0 || w % nnz != 0 || vec_stride < 1) return -1;
  if (dtype < NM_OR_F16 || dtype > NM_OR_F32 || !out_f32) return -1;
  const long long K = (long long)(w / nnz) * m;
  float* acc = out_f32;
  for (int r = 0; r < h; ++r) acc[r] = 0.0f;
  for (int c = 0; c < w; ++c) {
    const long long g = c / nnz;
    const long long pos = g * m + (long long)mat_index[c];
    const float x = pos < K ? load_elem(vec, (size_t)(pos * vec_stride), dtype) : 0.0f;
    const size_t base = (size_t)c * (size_t)h;
    for (int r = 0; r < h; ++r) acc[r] = fmaf(load_elem(mat_data, base + (size_t)r, dtype), x, acc[r]);
  }
  if (out) {
    for (int r = 0; r < h; ++r) {
      if (dtype == NM_OR_F16) ((uint16_t*)out)[r] = nm_oracle_f32_to_f16(acc[r]);
      else if (dtype == NM_OR_BF16) ((uint16_t*)out)[r] = nm_oracle_f32_to_bf16(acc[r]);
      else ((float*)out)[r] = acc[r];
    }
  }
  return 0;
}

/*
 * Faster fp16 variant for timing the CPU baseline: identical arithmetic and
 * order, with the fp16 -> fp32 conversion through a 64 K-entry table built
 * from nm_oracle_f16_to_f32.
 */
static float g_f16_table[65536];
static int g_f16_table_ready = 0;

void nm_oracle_init_tables(void) {
  if (g_f16_table_ready) return;
  for (uint32_t i = 0; i < 65536u; ++i) g_f16_table[i] = nm_oracle_f16_to_f32((uint16_t)i);
  g_f16_table_ready = 1;
}

int nm_oracle_gemv_f16_fast(const uint16_t* vec, const uint16_t* mat_data, const uint8_t* mat_index,
                            float* out_f32, uint16_t* out, int h, int w, int nnz, int m) {
  if (h <= 0 || w <= 0 || nnz <= 0 || m <= 0 || w % nnz != 0 || !out_f32) return -1;
  nm_oracle_init_tables();
  const long long K = (long long)(w / nnz) * m;
  float* acc = out_f32;
  for (int r = 0; r < h; ++r) acc[r] = 0.0f;
  for (int c = 0; c < w; ++c) {
    const long long pos = (long long)(c / nnz) * m + (long long)mat_index[c];
    const float x = pos < K ? g_f16_table[vec[pos]] : 0.0f;
    const uint16_t* row = mat_data + (size_t)c * (size_t)h;
    for (int r = 0; r < h; ++r) acc[r] = fmaf(g_f16_table[row[r]], x, acc[r]);
  }
  if (out)
    for (int r = 0; r < h; ++r) out[r] = nm_oracle_f32_to_f16(acc[r]);
  return 0;
}
