// roofline_probe.hip — measurement-only kernel: a plain streaming read.
//
// Not part of the GEMV's C ABI (it has no counterpart in the reference). The
// microbenchmark uses it to measure what one launch of a pure HBM read can
// achieve on this GPU for a given byte count and grid, i.e. the practical
// ceiling for the bandwidth-bound GEMV, and as the known-size kernel for
// calibrating the FETCH_SIZE counter. Each workgroup reads a contiguous slice
// with 16-byte non-temporal loads, U per lane in flight, and folds the words
// into one value that is stored only if it equals a sentinel (never, for the
// data the probe uses), so the loads cannot be removed.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ p, long long n16,
                                                          long long per_block, unsigned* __restrict__ sink) {
  const long long b0 = (long long)blockIdx.x * per_block;
  long long b1 = b0 + per_block;
  if (b1 > n16) b1 = n16;
  unsigned acc = 0;
  for (long long i = b0 + threadIdx.x; i < b1; i += 256LL * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long j = i + 256LL * u;
      v[u] = j < b1 ? __builtin_nontemporal_load(p + j) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}
// The GEMV's access pattern without its arithmetic: a row-major [R, C16]
// matrix of 16-byte words read in column stripes of SW words (workgroup b:
// stripe b % tiles, rows (b / tiles) * R / splits onward), 256 lanes, U rows
// per lane in flight. Row addresses are clamped into the workgroup's range.
template <int SW, int U>
__global__ __launch_bounds__(256) void stripe_read_kernel(const u32x4* __restrict__ p, int R, int C16, int tiles,
                                                          int splits, unsigned* __restrict__ sink) {
  const int tile = (int)blockIdx.x % tiles;
  const int split = (int)blockIdx.x / tiles;
  const int rows = R / splits;
  const int r0 = split * rows;
  const int col = tile * SW + (int)(threadIdx.x % SW);
  constexpr int kRowsPerPass = 256 / SW;
  unsigned acc = 0;
  for (int r = r0 + (int)(threadIdx.x / SW); r < r0 + rows; r += kRowsPerPass * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int rr = min(r + u * kRowsPerPass, r0 + rows - 1);
      v[u] = __builtin_nontemporal_load(p + (size_t)rr * (size_t)C16 + col);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}
}  // namespace

// Reads a row-major [R, C16] matrix of 16-byte words in column stripes of
// `sw` words (8, 16, 32, 64 or 128: 128 B to 2 KB per row; the GEMV's 128- to
// 1024-row tiles read 256 B to 2 KB of fp16 weights) with (C16 / sw) * splits
// workgroups, 8 rows per lane in flight. R must be a multiple of splits; `sink` must hold
// one uint32 per workgroup. Returns a hipError_t (0 on success), or -1.
extern "C" int nm_probe_stripe_read(const void* data, int R, int C16, int sw, int splits, void* sink, void* stream) {
  if (!data || !sink || R <= 0 || C16 <= 0 || splits <= 0 || R % splits || ((uintptr_t)data & 15)) return -1;
  if ((sw != 8 && sw != 16 && sw != 32 && sw != 64 && sw != 128) || C16 % sw) return -1;
  const int tiles = C16 / sw;
  const dim3 grid((unsigned)(tiles * splits));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const u32x4* p = static_cast<const u32x4*>(data);
  unsigned* k = static_cast<unsigned*>(sink);
  switch (sw) {
    case 8: hipLaunchKernelGGL((stripe_read_kernel<8, 8>), grid, dim3(256), 0, s, p, R, C16, tiles, splits, k); break;
    case 16: hipLaunchKernelGGL((stripe_read_kernel<16, 8>), grid, dim3(256), 0, s, p, R, C16, tiles, splits, k); break;
    case 32: hipLaunchKernelGGL((stripe_read_kernel<32, 8>), grid, dim3(256), 0, s, p, R, C16, tiles, splits, k); break;
    case 64: hipLaunchKernelGGL((stripe_read_kernel<64, 8>), grid, dim3(256), 0, s, p, R, C16, tiles, splits, k); break;
    default: hipLaunchKernelGGL((stripe_read_kernel<128, 8>), grid, dim3(256), 0, s, p, R, C16, tiles, splits, k); break;
  }
  return (int)hipGetLastError();
}

// Reads `bytes` (a multiple of 16) from 16-byte aligned `data` with `blocks`
// workgroups and `u` (4, 8 or 16) loads in flight per lane. `sink` must hold
// `blocks` uint32. Returns a hipError_t (0 on success), or -1 for bad arguments.
extern "C" int nm_probe_stream_read(const void* data, long long bytes, int blocks, int u, void* sink,
                                    void* stream) {
  if (!data || !sink || bytes <= 0 || (bytes & 15) || ((uintptr_t)data & 15) || blocks <= 0) return -1;
  const long long n16 = bytes / 16;
  const long long per = (n16 + blocks - 1) / blocks;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const u32x4* p = static_cast<const u32x4*>(data);
  unsigned* k = static_cast<unsigned*>(sink);
  switch (u) {
    case 4: hipLaunchKernelGGL(stream_read_kernel<4>, dim3(blocks), dim3(256), 0, s, p, n16, per, k); break;
    case 8: hipLaunchKernelGGL(stream_read_kernel<8>, dim3(blocks), dim3(256), 0, s, p, n16, per, k); break;
    case 16: hipLaunchKernelGGL(stream_read_kernel<16>, dim3(blocks), dim3(256), 0, s, p, n16, per, k); break;
    default: return -1;
  }
  return (int)hipGetLastError();
}
