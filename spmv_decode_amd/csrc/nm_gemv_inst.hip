// nm_gemv_inst.hip — instantiates every kernel configuration of one element
// type (NM_INST_DTYPE = NM_DTYPE_F16 / _BF16 / _F32, set by the build), so the
// three element types compile in parallel.

#include "nm_gemv_kernel.h"

#ifndef NM_INST_DTYPE
#error "compile with -DNM_INST_DTYPE=<0|1|2>"
#endif

namespace nm_hip {

#define NM_KERNEL_V(TH, U, G, NT, NM, NORM, CARRY, SILU) \
  &nm_gemv_kernel<NM_INST_DTYPE, TH, U, G, NT, NM, NORM, CARRY, SILU>
// variants (Variant in nm_gemv_kernel.h): plain, norm, carried 8 / 16 / 1, SiLU-product input (SILUK: the
// kernel for single-matrix rows, nullptr for the pair)
#define NM_SILU_1(TH, U, G, NT) NM_KERNEL_V(TH, U, G, NT, 1, false, 0, true)
#define NM_SILU_2(TH, U, G, NT) nullptr
#define NM_ROW_N(TH, U, G, NT, NM)                                                                         \
  {NM_KERNEL_V(TH, U, G, NT, NM, false, 0, false), NM_KERNEL_V(TH, U, G, NT, NM, true, 0, false),         \
   NM_KERNEL_V(TH, U, G, NT, NM, true, 8, false),  NM_KERNEL_V(TH, U, G, NT, NM, true, 16, false),        \
   NM_KERNEL_V(TH, U, G, NT, NM, true, 1, false),  NM_SILU_##NM(TH, U, G, NT)}
#define NM_ROW_W(TH, U, G, NT, NM)                                                                 \
  {NM_KERNEL_V(TH, U, G, NT, NM, false, 0, false), NM_KERNEL_V(TH, U, G, NT, NM, true, 0, false), \
   nullptr, nullptr, nullptr, NM_SILU_##NM(TH, U, G, NT)}
#define NM_ROW(NM, TH, U, NT) \
  {{NM_ROW_N(TH, U, 1, NT, NM), NM_ROW_N(TH, U, 2, NT, NM), NM_ROW_W(TH, U, 4, NT, NM), NM_ROW_W(TH, U, 8, NT, NM)}},
#define NM_PLAIN_ROW(TH, U, NT) NM_ROW(1, TH, U, NT)
#define NM_PAIR_ROW(TH, U, NT) NM_ROW(2, TH, U, NT)

#define NM_SPMM_G(TH, U, NT, NB) \
  {&nm_spmm_kernel<NM_INST_DTYPE, TH, U, 1, NT, NB>, &nm_spmm_kernel<NM_INST_DTYPE, TH, U, 2, NT, NB>, \
   &nm_spmm_kernel<NM_INST_DTYPE, TH, U, 4, NT, NB>}
#define NM_SPMM_ROW(TH, U, NT) {{NM_SPMM_G(TH, U, NT, 2), NM_SPMM_G(TH, U, NT, 4), NM_SPMM_G(TH, U, NT, 8)}},

#if NM_INST_DTYPE == NM_DTYPE_F16
#define NM_PLAIN_TABLE kPlainKernelsF16
#define NM_PAIR_TABLE kPairKernelsF16
#define NM_SPMM_TABLE kSpmmKernelsF16
#elif NM_INST_DTYPE == NM_DTYPE_BF16
#define NM_PLAIN_TABLE kPlainKernelsBF16
#define NM_PAIR_TABLE kPairKernelsBF16
#define NM_SPMM_TABLE kSpmmKernelsBF16
#else
#define NM_PLAIN_TABLE kPlainKernelsF32
#define NM_PAIR_TABLE kPairKernelsF32
#define NM_SPMM_TABLE kSpmmKernelsF32
#endif

const KernelRow NM_PLAIN_TABLE[kNumConfigs] = {NM_PLAIN_CONFIGS(NM_PLAIN_ROW)};
const KernelRow NM_PAIR_TABLE[kNumDualConfigs] = {NM_PAIR_CONFIGS(NM_PAIR_ROW)};
const SpmmRow NM_SPMM_TABLE[kNumSpmmConfigs] = {NM_SPMM_CONFIGS(NM_SPMM_ROW)};

}  // namespace nm_hip
