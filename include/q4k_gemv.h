/*
 * q4k_gemv.h -- C ABI of the MI355X (gfx950) Q4_K matrix-vector product.
 *
 * Drop-in for ggml's "mmvq" path of GGML_OP_MUL_MAT with a Q4_K weight
 * (src0), an F32 activation of 1..8 columns (src1) and an F32 result (dst).
 * Every entry point takes plain pointers and sizes, returns a q4k_status and
 * never throws or aborts.  All device work is enqueued on the caller's HIP
 * stream (passed as void *, NULL = the null stream) with no host
 * synchronisation, like the reference, which runs on ctx.stream().
 *
 * Memory: src0, src1 and dst are caller-owned device buffers.  Most calls
 * allocate nothing: the activation is quantised inside the GEMV launch.
 * q4k_mul_mat_vec_q and q6k_mul_mat_vec_q do allocate when the activation
 * does not fit one workgroup's LDS and no workspace is passed: a
 * stream-ordered temporary (hipMallocAsync/hipFreeAsync, the counterpart of
 * ggml's ctx.pool()) for the Q8_1 copy.  A caller with a pool (as ggml has)
 * should pass a workspace: it also speeds up several long columns.
 *
 * Threading: entry points may be called from any host thread; per-device
 * state is initialised once under a lock.  Calls that share a stream are
 * ordered by it.
 */
#ifndef Q4K_GEMV_H
#define Q4K_GEMV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
typedef enum q4k_status {
    Q4K_OK = 0,
    /* The shape or layout is outside what this path implements; the caller
     * falls back to another implementation.  Counterpart of the reference's
     * simple_ok gate, which routes such cases to the generic kernel
     * (kernels/mmvq.cu:540-545, :585-591). */
    Q4K_EUNSUPPORTED = 1,
    /* Invalid argument (null pointer, K not a multiple of 256, more than 8
     * columns, inconsistent strides).  The reference aborts on these with
     * GGML_ASSERT (kernels/mmvq.cu:393-394, :669-684). */
    Q4K_EINVAL = 2,
    /* A HIP runtime call or kernel launch failed; q4k_last_hip_error() gives
     * the hipError_t.  The reference leaves launches unchecked
     * (kernels/mmvq.cu:563-584). */
    Q4K_EHIP = 3,
    /* The stream-ordered temporary (or host memory) could not be allocated. */
    Q4K_ENOMEM = 4,
    /* A file could not be opened, read or mapped (GGUF reader). */
    Q4K_EIO = 5,
    /* A file is not a valid GGUF v2/v3 file (GGUF reader). */
    Q4K_EFORMAT = 6,
    /* q4k_mul_mat_vec_q_noalloc: q4k_q8_1_bytes(ne00, ne11) exceeds its
     * fixed device scratch (Q4K_NOALLOC_SCRATCH_BYTES); nothing was
     * launched. */
    Q4K_ESCRATCH = 7
} q4k_status;

/* ggml type ids used in descriptors (values of ggml's enum ggml_type) */
#define Q4K_GGML_TYPE_F32 0
#define Q4K_GGML_TYPE_Q8_1 9
#define Q4K_GGML_TYPE_Q4_K 12
#define Q4K_GGML_TYPE_Q6_K 14
#define Q4K_GGML_TYPE_I32 26  /* MUL_MAT_ID expert ids */

#define Q4K_QK_K 256            /* weights per Q4_K super-block */
#define Q4K_BLOCK_Q4_K_BYTES 144 /* d, dmin (fp16), scales[12], qs[128]; kernels/2pack.cu:6 */
#define Q4K_BLOCK_Q8_1_BYTES 36  /* ds (half2), qs[32]; kernels/2pack.cu:7 */
#define Q4K_BLOCK_Q6_K_BYTES 210 /* ql[128], qh[64], scales[16] (int8), d (fp16) */
#define Q4K_MATRIX_ROW_PADDING 512 /* K padding of the Q8_1 temp; kernels/mmvq.cu:728 */
#define Q4K_MAX_BATCH 8         /* MMVQ_MAX_BATCH_SIZE; kernels/mmvq.cu:394 */

/* The subset of ggml_tensor the op reads: type, ne[4] (elements per dim),
 * nb[4] (bytes per step in each dim), data (device pointer). */
typedef struct q4k_tensor {
    int32_t type;
    int64_t ne[4];
    size_t nb[4];
    void *data;
} q4k_tensor;

/* GLU ops of the fused epilogue (values of ggml's enum ggml_glu_op) */
#define Q4K_GLU_OP_GEGLU 1      /* up * gelu(gate), tanh form */
#define Q4K_GLU_OP_SWIGLU 2     /* up * silu(gate) */
#define Q4K_GLU_OP_SWIGLU_OAI 3 /* silu_1.702(min(gate, 7)) * (1 + clamp(up, -7, 7)) */

/* Fused epilogue of a one-column product, device pointers: the counterpart
 * of ggml_cuda_mm_fusion_args_device (kernels/mmvq.cu:692-715).  With it,
 * dst[r] = up + x_bias[r], where up = row r of src0 times src1; with a gate
 * weight, dst[r] = glu(up + x_bias[r], g + gate_bias[r]) where g = row r of
 * the gate times src1 (kernels/mmvq.cu:309-336).  NULL members are absent. */
typedef struct q4k_fusion {
    const float *x_bias;    /* ne01 floats */
    const void *gate;       /* same type, shape and row stride as src0 */
    const float *gate_bias; /* ne01 floats, used only with a gate */
    int32_t glu_op;         /* Q4K_GLU_OP_*, used only with a gate */
} q4k_fusion;

/* ggml-descriptor form (ggml_cuda_mm_fusion_args_host): F32 bias tensors of
 * ne[0] == dst->ne[0], a gate tensor of src0's type and strides. */
typedef struct q4k_fusion_args {
    const q4k_tensor *x_bias;
    const q4k_tensor *gate;
    const q4k_tensor *gate_bias;
    int32_t glu_op;
} q4k_fusion_args;

/* ----------------------------------------------------------------- misc */
int32_t q4k_version(void);
const char *q4k_strerror(int status);
/* hipError_t of the most recent Q4K_EHIP on the calling thread (0 if none) */
int32_t q4k_last_hip_error(void);

/* Bytes of the Q8_1 activation buffer for ne11 columns of ne10 values:
 * ne11 * pad(ne10, 512) / 32 * 36.  Same size as the reference's pool
 * allocation (kernels/mmvq.cu:728-729).  0 for negative sizes and for
 * ne10 > 2^40 or ne11 > 2^16, whose byte count could overflow. */
size_t q4k_q8_1_bytes(int64_t ne10, int64_t ne11);

/* ------------------------------------------------------------ entry points */

/* F32 -> Q8_1 activation quantiser for the 2-D case.  Replaces
 * quantize_row_q8_1_cuda(x, NULL, vy, type, ne00, s01, s02, s03, ne0,
 * ne1, 1, 1, stream) as called at kernels/mmvq.cu:734.
 *   x:    ne1 columns of ne00 floats, column stride s01 floats
 *   vy:   ne1 * ne0/32 block_q8_1, column after column; values at index
 *         >= ne00 quantise as 0 (ne0 = padded length, multiple of 32)
 * Per 32 values: d = amax/127, q = round(x/d) (0 if amax == 0),
 * ds = (half(d), half(sum x)). */
int q4k_quantize_row_q8_1(const float *x, void *vy, int64_t ne00, int64_t s01, int64_t ne0,
                          int64_t ne1, void *stream);

/* dst = src0 (Q4_K, ne01 x ne00) * src1 (F32, ne00 x ne11).  Replaces
 * ggml_cuda_mul_mat_vec_q(ctx, src0, src1, ids=NULL, dst, fusion=NULL)
 * (kernels/mmvq.cu:666-762) for the 2-D case.
 *   src0: ne01 rows, row stride nb01 bytes (multiple of 144), 16-B aligned
 *   src1: ne11 columns of ne00 floats, column stride nb11 bytes
 *   dst:  ne11 columns of ne01 floats, column stride nb1 bytes
 * ne00 must be a multiple of 256 and 1 <= ne11 <= 8 (ne01 == 0 or ne11 == 0
 * is an empty product and returns Q4K_OK).  The activation is quantised to
 * Q8_1 inside the GEMV launch when it fits one workgroup's LDS; otherwise
 * through a Q8_1 buffer: `workspace` (at least q4k_q8_1_bytes(ne00, ne11)
 * bytes, 4-B aligned) or, when NULL, a stream-ordered temporary.  With a
 * workspace of that size the buffer is also used, in a quantisation launch
 * of its own as the reference does, when ne00 * ne11 > 40960 (several long
 * columns, which every workgroup would otherwise quantise in full) and the
 * launch is not a K-split kernel (those quantise inside the launch; three or
 * four columns of 8193..16384 values run one).  Both routes give the same
 * bits. */
int q4k_mul_mat_vec_q(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01,
                      const float *src1, int64_t ne11, int64_t nb11, float *dst, int64_t nb1,
                      void *workspace, size_t workspace_bytes, void *stream);

/* Allocation-free form of q4k_mul_mat_vec_q (same arguments without the
 * workspace, same results bit for bit).  No counterpart in the reference:
 * it is for callers that cannot allocate device memory -- code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.  It
 * calls no hipMalloc/hipFree or allocating library routine; the Q8_1 copy
 * of the activation, when the route needs one, goes to a file-scope device
 * scratch of Q4K_NOALLOC_SCRATCH_BYTES that each GPU holds until the process
 * ends.  Limit: q4k_q8_1_bytes(ne00, ne11) <= Q4K_NOALLOC_SCRATCH_BYTES
 * (8 columns of up to 116224 values each, one column of up to 931840),
 * otherwise Q4K_ESCRATCH.  All calls on one GPU share its scratch: calls
 * that overlap in time on one GPU (different streams or host threads
 * without ordering between them) race; serialise them. */
#define Q4K_NOALLOC_SCRATCH_BYTES ((size_t)1 << 20)
int q4k_mul_mat_vec_q_noalloc(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01,
                              const float *src1, int64_t ne11, int64_t nb11, float *dst, int64_t nb1,
                              void *stream);

/* Row-slice GEMV on an already-quantised activation.  Replaces
 * ggml_cuda_op_mul_mat_vec_q(ctx, src0, src1, dst, src0_dd_i, src1_ddf_i,
 * src1_ddq_i, dst_dd_i, row_low, row_high, src1_ncols,
 * src1_padded_row_size, stream) (kernels/mmvq.cu:764-793), the per-device
 * call of ggml's split-mode-row multi-GPU matmul.
 *   src0_dd_i:   rows [row_low, row_high) of the Q4_K weight, contiguous
 *                (ne00/256 blocks per row), 16-B aligned
 *   src1_ddq_i:  src1_ncols columns of block_q8_1, column stride
 *                src1_padded_row_size/32 blocks
 *   dst_dd_i:    dst_dd_i[c*nrows_dst + r] for r < row_high-row_low
 * As in the reference, nrows_dst is ne0 on the device that holds the whole
 * result and row_high-row_low elsewhere (kernels/mmvq.cu:780-782). */
int q4k_op_mul_mat_vec_q(const void *src0_dd_i, int64_t ne00, int64_t row_low, int64_t row_high,
                         const void *src1_ddq_i, int64_t src1_ncols,
                         int64_t src1_padded_row_size, float *dst_dd_i, int64_t nrows_dst,
                         void *stream);

/* ggml-descriptor form of q4k_mul_mat_vec_q / q6k_mul_mat_vec_q: the
 * signature of ggml_cuda_mul_mat_vec_q (kernels/mmvq.cu:666-668) with
 * ggml_tensor replaced by q4k_tensor and the backend context by (workspace,
 * stream).  src0->type selects the weight format (Q4K_GGML_TYPE_Q4_K or
 * Q4K_GGML_TYPE_Q6_K, the reference's type switch at kernels/mmvq.cu:536,
 * :600-605; any other type returns Q4K_EUNSUPPORTED).
 * Checks the reference's assertions: src1/dst F32 (:669-670), nb00 == block
 * size, nb10 == 4, nb0 == 4 (:681-683), ne10 == ne00, ne0 == ne01, ne1 == ne11.
 * Channels and samples (dims 2 and 3) broadcast as in ggml's MUL_MAT:
 * dst channel c, sample s uses src0 matrix (c / (ne12/ne02), s / (ne13/ne03))
 * and src1 channel c, sample s (kernels/mmvq.cu:174-180, :739-755), all in
 * one launch.  With ids (I32, GGML_OP_MUL_MAT_ID for one token, ne12 == 1,
 * kernels/mmvq.cu:675): dst column j = src0 matrix ids[j] times src1 column
 * j % ne11; the ids are read on the device, and an id outside [0, ne02)
 * yields a zero column.
 * fusion (may be NULL) adds the bias / gate + GLU epilogue of
 * q4k_mul_mat_vec_q_fused under the reference's checks (:694-714): one dst
 * column per channel (dst->ne[1] == 1, or with ids dst->ne[2] == 1), F32
 * biases of dst->ne[0] values (with ids one row per src0 matrix), a gate of
 * src0's type, shape and strides; biases are indexed with dst's strides in
 * the dimensions the launch walks (other layouts: Q4K_EUNSUPPORTED). */
int q4k_ggml_mul_mat_vec_q(const q4k_tensor *src0, const q4k_tensor *src1, const q4k_tensor *ids,
                           q4k_tensor *dst, const q4k_fusion_args *fusion, void *workspace,
                           size_t workspace_bytes, void *stream);

/* One-column product with the fused epilogue (bias, gate + GLU): the
 * has_fusion instantiation of the reference's mul_mat_vec_q
 * (kernels/mmvq.cu:150-344, launched with fusion for ncols_dst == 1,
 * :697-698).  src0_type is Q4K_GGML_TYPE_Q4_K or Q4K_GGML_TYPE_Q6_K; src0
 * as for q4k_mul_mat_vec_q / q6k_mul_mat_vec_q (the gate with the same
 * alignment), src1 one column of ne00 floats, dst ne01 floats, biases 4-byte
 * aligned.  The gate is streamed beside src0 in the same launch, so both
 * products share one pass over the activation.  GLU ops other than
 * Q4K_GLU_OP_* return Q4K_EUNSUPPORTED (ggml runs those unfused). */
int q4k_mul_mat_vec_q_fused(int32_t src0_type, const void *src0, int64_t ne00, int64_t ne01,
                            int64_t nb01, const float *src1, const q4k_fusion *fusion, float *dst,
                            void *stream);

/* Parity probe: the int32 sub-block sums of the product, computed with the
 * GEMV kernel's own lane mapping and dot routines.
 *   sqq[(c*ne01 + r)*(ne00/32) + s] = sum over sub-block s of q4 * q8
 *   sq[c*(ne00/32) + s]            = sum over sub-block s of q8
 * q8_1 holds ncols columns of block_q8_1 with column stride stride_col_y
 * blocks.  These are the quantities of kernels/vecdotq.cuh:469-478 summed
 * over the lanes that share a sub-block. */
int q4k_subblock_sums(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01,
                      const void *q8_1, int64_t ncols, int64_t stride_col_y, int32_t *sqq,
                      int32_t *sq, void *stream);

/* Parity form of q4k_mul_mat_vec_q: the same routes, geometry and kernels,
 * in their variant that also stores the int32 sums it forms -- the
 * quantities of kernels/vecdotq.cuh:469-478 (dot1 per sub-block, summed over
 * the lanes that share it) and the activation sums the min term uses:
 *   sums[(c*ne01 + r)*(ne00/32) + s] = sum over sub-block s of q4 * q8
 *   sq[c*(ne00/32) + s]             = sum over sub-block s of q8
 * dst receives the product, bit for bit what q4k_mul_mat_vec_q writes.
 * Only launch shapes the automatic geometry picks have this variant (a
 * geometry override can return Q4K_EUNSUPPORTED).  No counterpart in the
 * reference; for parity tests. */
int q4k_mul_mat_vec_q_sums(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01,
                           const float *src1, int64_t ne11, int64_t nb11, float *dst, int64_t nb1,
                           void *workspace, size_t workspace_bytes, int32_t *sums, int32_t *sq,
                           void *stream);

/* ------------------------------------------------------------- Q6_K ---- */

/* dst = src0 (Q6_K, ne01 x ne00) * src1 (F32, ne00 x ne11): the Q6_K case of
 * ggml_cuda_mul_mat_vec_q (kernels/mmvq.cu:600-605 dispatches
 * mul_mat_vec_q<GGML_TYPE_Q6_K>, whose per-block dot product is
 * kernels/vecdotq.cuh:867-891 with :580-600).  Arguments, layout rules and
 * statuses as q4k_mul_mat_vec_q, except: src0 rows are block_q6_K (210 bytes
 * per 256 weights, nb01 a multiple of 210) and src0 needs 2-byte alignment.
 * Per block the product is d * sum over 16-weight groups g of
 * d8(g/2) * scales[g] * S_g, S_g = sum of (q - 32) * q8 (int32, exact). */
int q6k_mul_mat_vec_q(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01,
                      const float *src1, int64_t ne11, int64_t nb11, float *dst, int64_t nb1,
                      void *workspace, size_t workspace_bytes, void *stream);

/* Row-slice Q6_K GEMV on an already-quantised activation: the Q6_K case of
 * ggml_cuda_op_mul_mat_vec_q (kernels/mmvq.cu:764-793); arguments as
 * q4k_op_mul_mat_vec_q with src0_dd_i holding ne00/256 block_q6_K per row. */
int q6k_op_mul_mat_vec_q(const void *src0_dd_i, int64_t ne00, int64_t row_low, int64_t row_high,
                         const void *src1_ddq_i, int64_t src1_ncols,
                         int64_t src1_padded_row_size, float *dst_dd_i, int64_t nrows_dst,
                         void *stream);

/* Parity probe of the Q6_K GEMV: the int32 sums S_g over every 16-weight
 * scale group g of (q - 32) * q8, computed with the GEMV kernel's lane map,
 * activation staging and dot routine:
 *   s16[(c*ne01 + r)*(ne00/16) + g]
 * These are the dp4a sums of kernels/vecdotq.cuh:589-593 (vi - 32 against
 * u) summed over the four lanes that share a scale. */
int q6k_group_sums(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const void *q8_1,
                   int64_t ncols, int64_t stride_col_y, int32_t *s16, void *stream);

/* Parity form of q6k_mul_mat_vec_q (as q4k_mul_mat_vec_q_sums): the
 * production kernels' int32 group sums S_g of (q - 32) * q8,
 *   s16[(c*ne01 + r)*(ne00/16) + g]
 * (kernels/vecdotq.cuh:589-593 summed over the lanes sharing a scale), and
 * dst bit for bit what q6k_mul_mat_vec_q writes.  No counterpart in the
 * reference; for parity tests. */
int q6k_mul_mat_vec_q_sums(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01,
                           const float *src1, int64_t ne11, int64_t nb11, float *dst, int64_t nb1,
                           void *workspace, size_t workspace_bytes, int32_t *s16, void *stream);

/* Launch geometry q6k_mul_mat_vec_q would use (the out[] fields of
 * q4k_gemv_geometry; out[6] 1 tile kernel, 4 matrix-core kernel, 5 K-split
 * kernel, 6 matrix-core kernel reading its A operand from the Q8_1 buffer;
 * out[7] = weight groups in flight per wave). */
int q6k_gemv_geometry(int64_t ne00, int64_t ne01, int64_t ne11, int32_t out[8]);

/* The same for the pre-quantised route (as q4k_gemv_geometry_q8_1).  No
 * counterpart in the reference; for tests and benchmarks. */
int q6k_gemv_geometry_q8_1(int64_t ne00, int64_t ne01, int64_t ne11, int32_t out[8]);

/* The same for a one-column Q6_K launch with the fused epilogue (as
 * q4k_gemv_geometry_fused).  No counterpart in the reference; for tests and
 * benchmarks. */
int q6k_gemv_geometry_fused(int64_t ne00, int64_t ne01, int32_t with_gate, int32_t out[8]);

/* Launch geometry q4k_mul_mat_vec_q would use on the current device:
 * out[0] rows per wave tile (tile kernel), out[1] waves per workgroup,
 * out[2] workgroups, out[3] LDS bytes requested per workgroup, out[4] columns per
 * launch, out[5] 1 when the activation is quantised inside the GEMV launch,
 * out[6] kernel (1 tile, 2 block-per-lane, 3 coalesced block kernel, 4
 *        matrix-core kernel: tiles of 16 rows on v_mfma_i32_16x16x64_i8,
 *        5 K-split kernel: the waves of a workgroup split each row's
 *        super-blocks and quantise their own slice of the activation,
 *        6 matrix-core kernel reading its A operand from the Q8_1 buffer
 *        (pre-quantised route only)),
 * out[7] rows per wave step.  Where q4k_mul_mat_vec_q quantises into a
 * Q8_1 copy first for kernel 6, out[5] is 0 and the rest describes that
 * launch; the choice made with a workspace for long activations
 * (q4k_mul_mat_vec_q, workspace) is not modelled. */
int q4k_gemv_geometry(int64_t ne00, int64_t ne01, int64_t ne11, int32_t out[8]);

/* The same for the pre-quantised route: the launch q4k_op_mul_mat_vec_q
 * makes on a Q8_1 activation, and q4k_mul_mat_vec_q after quantising into
 * its workspace (out[5] is 0).  No counterpart in the reference; for tests
 * and benchmarks. */
int q4k_gemv_geometry_q8_1(int64_t ne00, int64_t ne01, int64_t ne11, int32_t out[8]);

/* The same for a one-column Q4_K launch with the fused epilogue, as
 * q4k_mul_mat_vec_q_fused makes it on a 16-byte aligned F32 activation:
 * with_gate != 0 a gate weight and the GLU, else a bias only.  No
 * counterpart in the reference; for tests and benchmarks. */
int q4k_gemv_geometry_fused(int64_t ne00, int64_t ne01, int32_t with_gate, int32_t out[8]);

/* Tuning override of the launch geometry for every later call in the
 * process: rows per wave tile of the tile kernel (1, 2, 4), waves per
 * workgroup (tile kernel: 1..8 selects the 8-wave, 9..16 the 16-wave
 * variant; reduced to 8 where 16 would not fit the registers), the number
 * of workgroups and the kernel (1 tile kernel, 2 block-per-lane, 3
 * coalesced block kernel where they apply, 4 matrix-core kernel for
 * products without an epilogue, 5 K-split kernel for one 16-byte aligned
 * F32 column of rows of up to 8 groups of 4096 values: rows_per_tile is
 * then its rows per wave step (1, 4, 8, 16; rows of other lengths than 4096
 * and 8192: 8 or 16), waves_per_wg 4, 8 or 16 (at least the rows per step;
 * other lengths: 8 or 16), and the pipeline override's slots its tiles in
 * flight (1..4; 3 and 4 for rows of 4096 values and 1, 4 or 8 rows per
 * step; other lengths 1 or 2); for two to four aligned F32 columns the
 * several-column K-split kernel (Q4_K and Q6_K): rows_per_tile 8 (two
 * columns, or four where the tile kernel would launch them two by two) or
 * 4, waves_per_wg 4, 8 or 16 (at least the rows per step), slots 1 or 2,
 * and with three or four columns of 4096 or 8192 values the pipeline
 * override's prologue 2 quantises the activation per wave in registers, any
 * other value once per workgroup into LDS (other lengths: always the
 * latter), 6 matrix-core kernel with its A operand read
 * from the Q8_1 buffer, for products of up to 8 columns on the
 * pre-quantised route; Q6_K: 4 the matrix-core kernel, 5 the K-split
 * kernel as for Q4_K (4, 8 or 16 rows per step), any other value the tile
 * kernel); 0 restores the automatic
 * choice.  Nothing is read from the environment: until this is called the
 * geometry is automatic.  Not part of the reference interface: a
 * benchmarking knob (ggml's counterpart is editing the compile-time tables
 * of kernels/mmvq.cu:95-147). */
int q4k_set_geometry_override(int32_t rows_per_tile, int32_t waves_per_wg, int32_t workgroups,
                              int32_t kernel);

/* Tuning override of the tile kernels' pipeline for every later call in the
 * process: weight groups in flight per wave (1, 2, 4 or 8; Q6_K uses 1 or 2;
 * the K-split kernel 1 to 4; 0 = automatic) and when the first weight
 * loads are issued relative to the activation quantisation (0 = the first
 * two groups before it, 1 = all
 * after, 2 = all before, 3 = one before; -1 = automatic; the long-row
 * K-split kernels: 2 = every group's slice quantised before the first
 * step, 0, 1, 3 = each group's just before the first step that reads it;
 * the several-column K-split kernel at three or four columns of 4096 or
 * 8192 values: 2 = quantised per wave in registers, else once per
 * workgroup).  Values a kernel
 * has no variant for fall back to the automatic choice.  Not part of the
 * reference interface: a benchmarking knob. */
int q4k_set_pipeline_override(int32_t slots, int32_t prologue);

/* A plain streaming read of `bytes` (< 2^31) of device memory: the ceiling
 * the GEMV is measured against, not part of its path.  workgroups x
 * waves_per_wg (4, 8, 16) waves, wave w reading bytes [w*bytes_per_wave,
 * +bytes_per_wave) (a multiple of 1024; past the buffer: zeros) with 16-byte
 * loads, loads_in_flight (1, 2, 4, 8) 1-KB load instructions issued
 * together; each wave stores an xor of its data in sink[w] (sink holds
 * workgroups * waves_per_wg words).  No counterpart in the reference: a
 * measurement tool for bench.py. */
int q4k_read_probe(const void *src, size_t bytes, int32_t workgroups, int32_t waves_per_wg,
                   int32_t bytes_per_wave, int32_t loads_in_flight, uint32_t *sink, void *stream);

/* ------------------------------------------------------------ host side */

/* Host Q4_K quantiser: nrows rows of n_per_row floats (multiple of 256)
 * into nrows * n_per_row/256 block_q4_K, using up to nthreads threads.
 * Replaces quantize_row_q4_K_ref row by row (ggml-quants.c, the weight
 * format the reference consumes); the byte layout is fixed by
 * kernels/vecdotq.cuh:785-807. */
int q4k_quantize_rows_q4_K(const float *src, void *dst, int64_t nrows, int64_t n_per_row,
                           int nthreads);

/* Host Q6_K quantiser: nrows rows of n_per_row floats (multiple of 256) into
 * nrows * n_per_row/256 block_q6_K, using up to nthreads threads.  Replaces
 * quantize_row_q6_K_ref row by row (ggml-quants.c); the byte layout is fixed
 * by kernels/vecdotq.cuh:867-891. */
int q4k_quantize_rows_q6_K(const float *src, void *dst, int64_t nrows, int64_t n_per_row,
                           int nthreads);

#ifdef __cplusplus
}
#endif

#endif /* Q4K_GEMV_H */
