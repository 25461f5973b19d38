/*
 * nmsparse_hip.h — C ABI of the MI355X (gfx950) shared-mask N:M sparse GEMV.
 *
 * The library (libnmsparse_hip.so) computes, for batch-1 decode,
 *
 *     out[r] = RNE_T( sum_{c < w} f32(mat_data[c, r]) * f32(vec[(c / nnz) * m + mat_index[c]]) )
 *
 * for r < h, with fp32 fused multiply-add accumulation, where
 *   - mat_data  is [w, h] row-major (h contiguous), element type T,
 *   - mat_index is [w / nnz, nnz] uint8, the kept positions inside each
 *     m-wide input group; one pattern is shared by all h output rows,
 *   - vec       is [1, K] with K = (w / nnz) * m, element stride vec_stride,
 *   - out       is [1, h], element type T (fp32 -> T rounds to nearest even).
 *
 * Reference interface replaced: the Triton launch wrapper
 * `nmsparse_spmv_forward_triton_ptx(vec, mat_data, mat_index, w, h,
 * BLOCK_WIDTH, NUM_THREADS, VEC_WIDTH, minibatch, vecNum, ...)`
 * (triton_spmv.py:229-318) together with the kernels it launches
 * (triton_spmv.py:56-115 generic, triton_spmv.py:149-214 A100). The
 * reference's zero-fill (triton_spmv.py:285), relaxed fp32 atomics
 * (triton_spmv.py:110-115, 209-214) and fp32 -> T cast (triton_spmv.py:318)
 * are folded into one launch: split-K partial sums go to a caller-provided
 * workspace and the last-arriving workgroup of each output tile reduces them
 * in a fixed order, so results are deterministic.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers (HBM). `stream` is a hipStream_t passed as
 *     void* (NULL = the default stream). Launches are asynchronous: nothing
 *     here synchronises, allocates device memory or reads device memory on
 *     the host, so the calls may be captured in a hipGraph.
 *   - Return value: 0 on success; a negative NM_ERR_* code for an argument
 *     the library rejects before launching; a positive hipError_t if the
 *     launch itself failed. nm_strerror() names every code.
 *   - Preconditions checked here (a subset of the reference wrapper's, which
 *     the Python layer re-checks with the reference's exception types):
 *     h > 0, h % 128 == 0 (triton_spmv.py:263-264); 0 < nnz <= m <= 256
 *     (uint8 positions); w > 0, w % nnz == 0 (triton_spmv.py:265-266);
 *     vec_stride >= 1; non-NULL pointers; 16-byte aligned mat_data and out
 *     base addresses; workspace_bytes >= nm_gemv_workspace_bytes(...).
 *   - A position with (c / nnz) * m + mat_index[c] >= K contributes 0 (the
 *     reference kernel would read outside vec there).
 *
 * Workspace layout: the first NM_TICKET_BYTES bytes hold uint32 arrival
 * counters that must be zero before the first call that uses the workspace
 * (allocate it zero-filled once); every launch leaves them zero again. The
 * rest holds fp32 split-K partial sums. Calls that share one workspace must be
 * ordered (same stream, or synchronised); overlapping calls on one workspace
 * race.
 */
#ifndef NMSPARSE_HIP_H
#define NMSPARSE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NM_TICKET_BYTES 65536

/* Negative status codes (positive codes are hipError_t values). */
#define NM_OK 0
#define NM_ERR_NULL_POINTER (-1)
#define NM_ERR_BAD_SHAPE (-2)        /* h, w, nnz, m or vec_stride out of range */
#define NM_ERR_H_NOT_MULTIPLE_128 (-3)
#define NM_ERR_W_NOT_MULTIPLE_NNZ (-4)
#define NM_ERR_MISALIGNED (-5)       /* mat_data or out not 16-byte aligned */
#define NM_ERR_WORKSPACE (-6)        /* workspace missing or too small */
#define NM_ERR_BAD_CONFIG (-7)       /* explicit config id / split count rejected */
#define NM_ERR_BAD_EPILOGUE (-8)     /* input-norm / residual / head-layout arguments rejected */
#define NM_ERR_STATIC_SCRATCH (-9)   /* launch needs more than NM_STATIC_SCRATCH_BYTES (static entry point) */

/* Element type codes for the *_ex entry point and nm_gemv_workspace_bytes. */
#define NM_DTYPE_F16 0
#define NM_DTYPE_BF16 1
#define NM_DTYPE_F32 2

/*
 * Bytes of workspace a call with these sizes needs (NM_TICKET_BYTES plus the
 * split-K partials of the configuration the library picks for the shape).
 * Replaces the reference's per-call `torch.zeros((1, h), float32)` scratch
 * (triton_spmv.py:285). Returns 0 for arguments nm_gemv_* would reject.
 */
size_t nm_gemv_workspace_bytes(int h, int w, int nnz, int m);

/*
 * Typed GEMV entry points. vec, mat_data and out share the element type.
 * Replace `nmsparse_spmv_forward_triton_ptx` (triton_spmv.py:229-318) for
 * vec.dtype == float16 / bfloat16 / float32 (triton_spmv.py:248-251); the
 * op layer `torch.ops.nmsparse.gemv` (src/spmv/nmsparse_op.py:77-96) calls
 * the fp16 one.
 */
int nm_gemv_f16(const void* vec, int vec_stride, const void* mat_data,
                const uint8_t* mat_index, void* out, void* workspace,
                size_t workspace_bytes, int h, int w, int nnz, int m,
                void* stream);
int nm_gemv_bf16(const void* vec, int vec_stride, const void* mat_data,
                 const uint8_t* mat_index, void* out, void* workspace,
                 size_t workspace_bytes, int h, int w, int nnz, int m,
                 void* stream);
int nm_gemv_f32(const void* vec, int vec_stride, const void* mat_data,
                const uint8_t* mat_index, void* out, void* workspace,
                size_t workspace_bytes, int h, int w, int nnz, int m,
                void* stream);

/*
 * Same computation with an explicit kernel configuration, for tuning sweeps
 * and tests of every configuration. config_id < 0 selects the library's own
 * choice; otherwise 0 <= config_id < nm_num_configs(). splits <= 0 lets the
 * library choose the split-K count for that configuration. Replaces the
 * reference's autotune search space (triton_spmv.py:40-55, 122-148), which
 * the harness reads back via `best_config` (microbench_triton_torchmv.py:271-297).
 * The workspace must then hold nm_gemv_workspace_bytes_ex(...) bytes.
 */
int nm_gemv_ex(int dtype, const void* vec, int vec_stride, const void* mat_data,
               const uint8_t* mat_index, void* out, void* workspace,
               size_t workspace_bytes, int h, int w, int nnz, int m,
               int config_id, int splits, void* stream);
size_t nm_gemv_workspace_bytes_ex(int h, int w, int nnz, int m, int config_id,
                                  int splits);

/*
 * Grouped launch: nprob (1..4) GEMVs that read the same vec (same K, nnz, m,
 * hence the same w) in one grid, e.g. the q, k and v projections of one
 * attention layer. Problem i reads mat_data[i] ([w, hs[i]]) and
 * mat_index[i] and writes out[i] ([1, hs[i]]); each result is what
 * nm_gemv_ex would compute for that problem with the same config_id and
 * splits (all problems share one configuration). No reference counterpart as
 * an entry point: it fuses the per-projection calls the reference makes, the
 * multi-problem launch planned for the fused wqkv projection of gpt-fast
 * (model.py:196-198, 219). Workspace: nm_gemv_grouped_workspace_bytes.
 */
size_t nm_gemv_grouped_workspace_bytes(int nprob, const int* hs, int w, int nnz, int m, int config_id,
                                       int splits);
int nm_gemv_grouped(int dtype, const void* vec, int vec_stride, int nprob, const void* const* mat_data,
                    const uint8_t* const* mat_index, void* const* out, const int* hs, void* workspace,
                    size_t workspace_bytes, int w, int nnz, int m, int config_id, int splits, void* stream);

/*
 * Gate/up pair with the SiLU-gated epilogue of a Llama/Qwen MLP: one launch
 * computes g = W_gate x and u = W_up x (each an N:M GEMV with its own
 * mat_index, both [w, h]) and writes out[r] = RNE_T(silu(g[r]) * u[r]) with
 * silu(g) = g / (1 + exp(-g)), all in fp32 before the single rounding.
 * Replaces `F.silu(w1(x)) * w3(x)` (model.py:255-256) when w1 and w3 are
 * N:M sparse. config_id indexes the pair configurations
 * (0 <= config_id < nm_num_gate_up_configs(), < 0: the library's choice).
 * Workspace: nm_gemv_gate_up_workspace_bytes.
 */
size_t nm_gemv_gate_up_workspace_bytes(int h, int w, int nnz, int m, int config_id, int splits);
int nm_gemv_gate_up_silu(int dtype, const void* vec, int vec_stride, const void* gate_data,
                         const uint8_t* gate_index, const void* up_data, const uint8_t* up_index, void* out,
                         void* workspace, size_t workspace_bytes, int h, int w, int nnz, int m,
                         int config_id, int splits, void* stream);
int nm_num_gate_up_configs(void);

/*
 * General launch descriptor: the grouped launch or the gate/up pair, plus the
 * fusions at the GEMV's edges that a decoder layer needs. No reference
 * counterpart as an entry point; each fusion replaces PyTorch operations of
 * the reference's decode step around the sparse Linear:
 *
 *  - norm_weight != NULL: the input is RMSNorm(vec) = vec * s * norm_weight
 *    with s = 1 / sqrt(mean(vec^2) + norm_eps), computed in fp32. The gather
 *    reads vec * norm_weight and s scales the finished sums, so the
 *    normalised activation is never stored or rounded. Replaces the
 *    RMSNorm before the q/k/v and gate/up projections (attention_norm /
 *    ffn_norm, model.py:182-187; RMSNorm, model.py:258-270). Requires vec_stride == 1, a 16-byte aligned
 *    vec and K * sizeof(element) a multiple of 16.
 *  - prob[i].residual != NULL: out = residual + result, added in fp32 before
 *    the single rounding (the residual adds, model.py:186-187). residual
 *    may be the same buffer as out (each element is read before it is
 *    written, by the same lane); it must not overlap vec.
 *  - heads (grouped kind only; head_dim a multiple of 64 dividing h and the
 *    configuration's tile of 8*th rows): rows are head_dim-wide heads.
 *    head_norm != NULL applies a per-head RMSNorm (weight [head_dim],
 *    head_norm_eps; Qwen3's q_norm / k_norm); rope != 0 then rotates each
 *    (even, odd) row pair of a head by the angle of position *pos
 *    (rope_table [pos_limit, head_dim / 2] pairs (cos, sin), fp32), the
 *    complex-multiply convention of model.py:310-322. A non-zero
 *    head_stride / elem_stride / pos_stride writes row r to
 *    out[(r / head_dim) * head_stride + (r % head_dim) * elem_stride
 *        + (*pos) * pos_stride] (elements), e.g. straight into a KV cache
 *    slot, replacing the cache update (KVCache.update, model.py:114-123); nothing is stored
 *    when *pos is outside [0, pos_limit). The residual is added last.
 *
 *  - Split-K carry between consecutive launches of a decoder layer (replaces
 *    the residual add after o_proj / down_proj, model.py:186-187, moved into
 *    the next launch): carry_out != NULL makes a producer, one plain GEMV
 *    (grouped kind, nprob 1, no norm, residual or heads; prob[0].out unused)
 *    that leaves its fp32 split partials [splits, h] in carry_out (splits as
 *    nm_gemv_launch_plan reports for the descriptor with carry_out set: with
 *    no handoff to pay for, a producer whose default plan would leave a
 *    quarter of the CUs idle takes 128-row tiles and more splits, at most 16)
 *    and reduces nothing. carry_in != NULL makes
 *    a consumer (norm_weight required, 16-byte aligned; K = the producer's h;
 *    m a multiple of 4) whose
 *    input is x = round(sum over the carry_splits (<= 16) partials, in split
 *    order, + vec): bit for bit what the producer with residual vec would
 *    have written. The consumer writes x to vec_out ([K], apart from vec and
 *    carry_in) and
 *    otherwise runs as with vec = x, except that the input norm's mean(x^2)
 *    is summed per split slice (a different fp32 summation order). Its plan
 *    puts whole groups of nnz columns, at most 512, spanning at most 1024
 *    positions of K, in each split; shapes that cannot are rejected with
 *    NM_ERR_BAD_EPILOGUE.
 *
 *  - Accumulated carry (the reference's relaxed fp32 atomic accumulation,
 *    triton_spmv.py:209-214, used as the medium between two launches; the
 *    order of the additions, hence the last bits of the sums, varies from run
 *    to run). carry_accumulate != 0 with carry_out:
 *      * a plain producer (as above) adds its partial tile into carry_out[0, :]
 *        ([h] fp32, zero before the launch) instead of writing its split's
 *        row; a consumer then reads it with carry_splits = 1;
 *      * the gate/up pair (with or without carry_in) becomes a producer too:
 *        it adds gate's and up's raw sums (the input norm's scale not applied)
 *        into carry_out[0, h) and [h, 2h) ([2h + 16] fp32, the sums zero
 *        before the launch) and stores its input's sum of squares in
 *        carry_out[2h + split] (one per split with a carried input, whose
 *        plan must then have at most 16 splits; the whole sum in
 *        carry_out[2h] otherwise; nothing without norm_weight); prob[0].out
 *        is unused. The pair is a producer only in this form.
 *    silu_in != NULL (grouped kind, nprob 1, no norm_weight or carry_in; vec
 *    unused and may be NULL): the input is x[k] = round(silu(s * G[k]) *
 *    (s * U[k])), G = silu_in[0, K), U = silu_in[K, 2K), s = 1 / sqrt(sum of
 *    silu_in[2K, 2K + silu_ssq_n) / silu_k + silu_eps) (s = 1 when silu_ssq_n
 *    is 0; silu_ssq_n <= 16; silu_in apart from every other buffer of the
 *    launch): the gate/up pair's epilogue, done where down_proj gathers its
 *    input. zero_buf != NULL ([zero_len] fp32, 16-byte aligned,
 *    zero_len a multiple of 4, apart from every other buffer of the launch)
 *    is cleared by the launch: the accumulator a later launch adds into. No
 *    reference counterpart for silu_in and zero_buf.
 *
 * For NM_KIND_GATE_UP, nprob is 2 (prob[0] gate, prob[1] up, same h); the
 * output, residual and h are prob[0]'s, and no heads fusion is allowed.
 * Workspace: nm_gemv_launch_workspace_bytes(desc) (0 if the shape is
 * rejected). Every other convention is that of the entry points above.
 */
#define NM_KIND_GROUPED 0
#define NM_KIND_GATE_UP 1

typedef struct nm_gemv_problem {
  const void* mat_data;        /* [w, h] */
  const uint8_t* mat_index;    /* [w / nnz, nnz] */
  void* out;                   /* [h] (or the heads layout base) */
  const void* residual;        /* NULL or [h] */
  const void* head_norm;       /* NULL or [head_dim] */
  long long head_stride;       /* heads layout, in elements (all 0: out[r]) */
  long long elem_stride;
  long long pos_stride;
  int h;
  int rope;                    /* 0 or 1 */
} nm_gemv_problem;

typedef struct nm_gemv_launch_desc {
  int dtype;                   /* NM_DTYPE_* */
  int kind;                    /* NM_KIND_* */
  int nprob;                   /* grouped: 1..4; gate/up: 2 */
  int vec_stride;
  const void* vec;             /* [1, K], K = (w / nnz) * m */
  const void* norm_weight;     /* NULL or [K] */
  float norm_eps;
  float head_norm_eps;
  int head_dim;
  int pos_limit;
  const long long* pos;        /* device int64 [1] */
  const float* rope_table;     /* device fp32 [pos_limit, head_dim / 2, 2] */
  int w, nnz, m;
  int config_id, splits;       /* as nm_gemv_ex (pair configs for the gate/up kind) */
  nm_gemv_problem prob[4];
  float* carry_out;            /* NULL or [splits, h] fp32: producer */
  const float* carry_in;       /* NULL or [carry_splits, K] fp32: consumer */
  void* vec_out;               /* consumer: [K] receives its finished input */
  int carry_splits;
  int carry_accumulate;        /* producer: 1 = add into carry_out (accumulated carry) */
  float* zero_buf;             /* NULL or [zero_len] fp32 cleared by the launch */
  int zero_len;
  const float* silu_in;        /* NULL or [2K + silu_ssq_n] fp32: the SiLU-product input */
  int silu_ssq_n;
  int silu_k;
  float silu_eps;
} nm_gemv_launch_desc;

size_t nm_gemv_launch_workspace_bytes(const nm_gemv_launch_desc* desc);
/* The plan of such a launch (only the kind, counts, sizes, config_id,
 * splits and whether carry_in and carry_out are set are read): configuration, splits,
 * workgroups, compressed rows per split and rows per chunk. */
int nm_gemv_launch_plan(const nm_gemv_launch_desc* desc, int* out_config_id, int* out_splits, int* out_blocks,
                        int* out_rows_per_split, int* out_chunk_rows);
int nm_gemv_launch(const nm_gemv_launch_desc* desc, void* workspace, size_t workspace_bytes, void* stream);

/*
 * nm_gemv_launch without a workspace argument: the launch's counters and
 * split-K partials live in a scratch array of NM_STATIC_SCRATCH_BYTES that the
 * library holds in static device memory, one copy per GPU for the life of the
 * process. No counterpart in the reference (whose scratch comes from the
 * caching allocator per call, triton_spmv.py:285): it is for callers that
 * cannot allocate device memory -- code that must not call hipMalloc, such as
 * hipGraph capture without a memory pool, tight serving loops and harnesses
 * that forbid allocation. It allocates nothing and frees nothing. Same
 * descriptor, results and checks as nm_gemv_launch (the same kernels and
 * plans, so outputs are bit-identical to it); a launch whose
 * nm_gemv_launch_workspace_bytes(desc) exceeds NM_STATIC_SCRATCH_BYTES is
 * rejected with NM_ERR_STATIC_SCRATCH before anything runs. The counters start
 * at zero and every launch leaves them zero. All calls on one GPU share its
 * array: calls that may overlap on one GPU (different streams without
 * ordering) race and must not be made. The first call on each GPU looks the
 * array's address up (hipGetSymbolAddress, which may load the library's device
 * code): make it outside graph capture. The stream's device is the one used.
 */
#define NM_STATIC_SCRATCH_BYTES (NM_TICKET_BYTES + (16 << 20))
int nm_gemv_launch_static(const nm_gemv_launch_desc* desc, void* stream);

/*
 * Small-batch SpMM: out[b, :] = W x[b, :] for 1 <= batch <= NM_MAX_BATCH
 * activation rows that share one pass over the packed weights (multi-token
 * decode, batched serving, short prefills). x rows are x_row_stride elements
 * apart with unit column stride; out rows out_row_stride elements apart.
 * config_id: 0..3 (th16_u4, th16_u8, th32_u4, th32_u8) or < 0 for the
 * library's choice. With the same config_id and splits as nm_gemv_ex, and at
 * most 1024 compressed columns per split (nm_spmm_plan reports the plan),
 * every output row is bit-identical to nm_gemv_ex of that row. No reference
 * counterpart: the reference op rejects rows != 1 (src/spmv/nmsparse_op.py:83-86,
 * triton_spmv.py:257-258) and its module runs such inputs through a dense
 * F.linear (src/spmv/nmsparse_linear.py:62-68).
 */
#define NM_MAX_BATCH 8
size_t nm_spmm_workspace_bytes(int batch, int h, int w, int nnz, int m, int config_id, int splits);
int nm_spmm(int dtype, const void* x, long long x_row_stride, int batch, const void* mat_data,
            const uint8_t* mat_index, void* out, long long out_row_stride, void* workspace,
            size_t workspace_bytes, int h, int w, int nnz, int m, int config_id, int splits, void* stream);
int nm_spmm_plan(int batch, int h, int w, int nnz, int m, int config_id, int splits, int* out_config_id,
                 int* out_splits, int* out_blocks, int* out_rows_per_block);

/*
 * Matrix-core SpMM: the same product for 1 <= batch <= NM_MC_MAX_BATCH rows
 * in one pass over the packed weights, fp16 and bf16 only
 * (v_mfma_f32_16x16x32_f16 / _bf16: fp32 accumulation, one rounding to the
 * element type at the end, like nm_spmm; the order of the sums differs, so
 * rows are not bit-identical to nm_gemv_ex). Meant for more than
 * NM_MAX_BATCH rows (prefill chunks, batched serving), where nm_spmm needs a
 * launch per 8 rows. x rows x_row_stride >= K elements apart, out rows
 * out_row_stride >= h apart; mat_data and out 16-byte aligned, workspace
 * 256-byte aligned with zeroed arrival counters (as nm_gemv_ex).
 * config_id: 0..2 (output tiles of 64, 128, 256 columns, weights staged
 * through registers), 3..5 (the same tiles, weights and gathered
 * activations loaded straight into a ring of LDS stages), or < 0 for the
 * library's choice; splits <= 0 likewise. No reference counterpart (the
 * reference op rejects rows != 1, src/spmv/nmsparse_op.py:83-86, and its
 * module runs them through a dense F.linear, src/spmv/nmsparse_linear.py:62-68).
 */
#define NM_MC_MAX_BATCH 128
size_t nm_spmm_mc_workspace_bytes(int batch, int h, int w, int nnz, int m, int config_id, int splits);
int nm_spmm_mc(int dtype, const void* x, long long x_row_stride, int batch, const void* mat_data,
               const uint8_t* mat_index, void* out, long long out_row_stride, void* workspace,
               size_t workspace_bytes, int h, int w, int nnz, int m, int config_id, int splits, void* stream);
int nm_spmm_mc_plan(int batch, int h, int w, int nnz, int m, int config_id, int splits, int* out_config_id,
                    int* out_splits, int* out_blocks, int* out_rows_per_block);

/*
 * The matrix-core SpMM of round(silu(gate) * up): nm_spmm_mc whose
 * activations are formed from the gate and up projections' outputs (rows
 * x_row_stride apart in both) at the gathered positions, in fp32 with one
 * rounding to the element type, as the GEMV gate/up pair's epilogue. The
 * workspace is nm_spmm_mc_workspace_bytes'. No reference counterpart (the
 * reference forms F.silu(w1(x)) * w3(x) in PyTorch before w2, model.py:255-256,
 * for one row at a time).
 */
int nm_spmm_mc_silu_mul(int dtype, const void* gate, const void* up, long long x_row_stride, int batch,
                        const void* mat_data, const uint8_t* mat_index, void* out, long long out_row_stride,
                        void* workspace, size_t workspace_bytes, int h, int w, int nnz, int m, int config_id,
                        int splits, void* stream);

/*
 * Several matrix-core SpMMs of the same activations in one grid: product i
 * (0 <= i < n <= NM_MC_MAX_GROUP) is out[i] = mat_data[i] / mat_index[i]
 * applied to every row of x, h[i] outputs, out rows out_row_stride[i] apart;
 * all products share x, batch, w, nnz and m (sibling Linears: q/k/v, gate/up)
 * and one tile width and split count. Each product's rows are those
 * nm_spmm_mc gives with the same config_id and splits. One gather launch for
 * every product's activations, one product launch. No reference counterpart
 * (the reference has no multi-row path; its benchmark runs each Linear on its
 * own, src/spmv/nmsparse_linear.py:62-68).
 */
#define NM_MC_MAX_GROUP 4
size_t nm_spmm_mc_group_workspace_bytes(int batch, int n, const int* h, int w, int nnz, int m, int config_id,
                                        int splits);
int nm_spmm_mc_group(int dtype, const void* x, long long x_row_stride, int batch, int n,
                     const void* const* mat_data, const uint8_t* const* mat_index, void* const* out,
                     const long long* out_row_stride, const int* h, void* workspace, size_t workspace_bytes,
                     int w, int nnz, int m, int config_id, int splits, void* stream);
int nm_spmm_mc_group_plan(int batch, int n, const int* h, int w, int nnz, int m, int config_id, int splits,
                          int* out_config_id, int* out_splits, int* out_blocks, int* out_rows_per_block);

/*
 * The gathered activations alone: out[r, c] = x[r, (c/nnz)*m + mat_index[c]]
 * for c < w, zero for out_row_stride > c >= w (fp16 / bf16; out 16-byte
 * aligned, out_row_stride a multiple of 8 and >= w rounded up to 8). With
 * it, more rows than NM_MC_MAX_BATCH are a plain GEMM of out [rows, w] and
 * mat_data [w, h] for a BLAS library (the Python layer uses hipBLASLt
 * through torch.matmul). No reference counterpart.
 */
int nm_gather_columns(int dtype, const void* x, long long x_row_stride, int rows, const uint8_t* mat_index, int w,
                      int nnz, int m, void* out, long long out_row_stride, void* stream);

/*
 * Configuration introspection. nm_config_describe writes a short text such as
 * "th32_u8" into buf (ids nm_num_configs() + j describe pair configuration j);
 * nm_gemv_plan reports the configuration and split count the library would
 * use for a single GEMV of a shape (config_id < 0: its own choice).
 */
int nm_num_configs(void);
int nm_config_describe(int config_id, char* buf, int buf_len);
int nm_gemv_plan(int h, int w, int nnz, int m, int config_id, int splits,
                 int* out_config_id, int* out_splits, int* out_blocks,
                 int* out_rows_per_block);

/* Human-readable text for a status code returned above. */
const char* nm_strerror(int code);

/*
 * Capture state of `stream` as the HIP runtime this library links reports it
 * (hipStreamGetCaptureInfo): *out_id receives the id of the graph capture in
 * progress on the stream, or 0 when the stream is not capturing. Returns 0 or
 * the hipError_t. No reference counterpart: the Python layer keys the
 * workspaces of launches recorded into a capture by this id, through the
 * runtime the library itself uses (whatever its soname).
 */
int nm_stream_capture_id(void* stream, unsigned long long* out_id);

/* ABI version of this header (bumped on any signature change). */
int nm_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* NMSPARSE_HIP_H */
