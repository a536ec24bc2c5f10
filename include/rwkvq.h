/*
 * rwkvq.h -- C ABI of librwkvq_hip.so, the MI355X (gfx950) group-affine
 * quantized-linear library.
 *
 * The reference (RafaelUI/rwkv-metal) reaches quantized arithmetic only through
 * the upstream MLX op API.  Each entry point below replaces one of those ops:
 *
 *   rq_quantize    <- mx.quantize(w, group_size, bits)            (affine mode)
 *                     called via nn.quantize at rwkv_metal/lora/finetune.py:88-89
 *                     and QuantizedLinear.from_linear at rwkv_metal/lora/lora.py:45-46
 *   rq_dequantize  <- mx.dequantize(w_q, scales, biases, group_size, bits)
 *                     tests/dev_pack_native_mlx.py:70, tests/dev_check_hybrid.py:13
 *   rq_qmm         <- mx.quantized_matmul(x, w_q, scales, biases, transpose, group_size, bits)
 *                     rwkv_metal/lora/rwkvq_native.py:120-122 (transpose=True, forward);
 *                     its VJP w.r.t. x (transpose=False) is the QLoRA backward
 *                     reached from nn.value_and_grad at rwkv_metal/lora/finetune.py:141
 *   rq_pack        <- _pack_codes_mlx / codec.pack_mlx_affine, rwkv_metal/lora/rwkvq_native.py:81-90
 *                     (codes -> MLX bitstream; executable form tests/dev_pack_native_mlx.py:38-57)
 *   rq_unpack      <- the inverse of that packing rule (rwkvq_native.py:18-33), i.e. the
 *                     code extraction inside mx.dequantize
 *   rq_embedding   <- nn.QuantizedEmbedding lookup (gather + mx.dequantize), target "emb"
 *                     of rwkv_metal/lora/finetune.py:42, used at rwkv_metal/model/rwkv7_x070.py:302
 *   rq_qmm_lora    <- LoRALinear.__call__ over a quantized base (rwkv_metal/lora/lora.py:58-63)
 *                     and its dX (finetune.py:141): the low-rank term fused into rq_qmm's
 *                     output stage
 *   rq_qlora       <- the same layer with x . A^T (or dY . B) computed inside the GEMM:
 *                     forward and dX each one launch
 *   rq_qlora_dx    <- its dX from the adapters as stored (no transposed copies)
 *   rq_lora_down   <- its x . A^T and the backward's dY . B (the same lines)
 *   rq_lora_grads  <- the backward's adapter gradients u^T x and dY^T z (the same
 *                     layer under nn.value_and_grad, rwkv_metal/lora/finetune.py:141)
 *   rq_sb6_dequantize / rq_sb6_to_affine
 *                  <- the .rwkvq (rwkv-quant sb6) base: RwkvqLinear's fused dequant
 *                     (rwkv_metal/lora/rwkvq_kernel.py) and RwkvqNativeLinear's repack into
 *                     the MLX layout (rwkv_metal/lora/rwkvq_native.py:49-113)
 *   rq_qmm_grouped <- several independent mx.quantized_matmul(transpose=True) nodes of one
 *                     lazy MLX graph evaluated together (e.g. tmix r/k/v projections,
 *                     rwkv_metal/model/rwkv7_x070.py:142-144); one launch for all of them
 *   rq_grouped_plan_* <- the same, with the launch schedule kept in device memory so that
 *                     any number of problems runs as one launch per call
 *
 * Layout (identical to MLX's): W is [rows, cols], cols (= in_features) is the
 * grouped and packed axis.  w_q is uint32[rows, cols*bits/32], each row an
 * LSB-first bitstream with code j at bits [j*bits, (j+1)*bits).  scales and
 * biases are [rows, cols/group_size] in scales' dtype; ŵ = scale*code + bias.
 *
 * Conventions: every pointer is a device pointer owned by the caller; nothing
 * is allocated; work is enqueued on `stream` (a hipStream_t, NULL = the
 * default stream) with no implicit synchronisation.  Row-major, contiguous.
 * Device pointers must be 16-byte aligned unless an entry point says otherwise.
 *
 * Return codes: RQ_OK (0); RQ_EINVAL (-1): bits not in {2,3,4,5,6,8},
 * group_size not in {32,64,128}, cols % group_size != 0, a negative size, a
 * NULL pointer or an unknown dtype; RQ_EALIGN (-2): a pointer not 16-byte
 * aligned; RQ_ELAUNCH (-3): the HIP launch failed; RQ_EUNSUPPORTED (-4): valid
 * arguments outside what the called entry point covers (the message names the
 * entry point that does).  rq_last_error() returns a
 * thread-local message describing the last non-zero return.
 *
 * Reentrant: calls from several host threads on different streams are safe.
 */
#ifndef RWKVQ_H
#define RWKVQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RWKVQ_ABI_VERSION 1

typedef enum { RQ_BF16 = 0, RQ_F16 = 1, RQ_F32 = 2 } rq_dtype;

enum { RQ_OK = 0, RQ_EINVAL = -1, RQ_EALIGN = -2, RQ_ELAUNCH = -3, RQ_EUNSUPPORTED = -4 };

/* ABI version of the loaded library (RWKVQ_ABI_VERSION). */
int rq_abi_version(void);

/* Thread-local description of the last non-zero return ("" if none). */
const char* rq_last_error(void);

/* mx.quantize, affine mode.  w: [rows, cols] in w_dt.  Writes w_q
 * uint32[rows, cols*bits/32] and scales/biases [rows, cols/group_size] in w_dt.
 * Per group: fp32 min/max; scale = max((max-min)/(2^bits-1), 1e-7), negated
 * unless |min| > |max|; the larger-magnitude extreme e becomes the bias and
 * scale = e/rint(e/scale) when rint(e/scale) != 0 (else bias = 0);
 * code = clip(rint((w-bias)/scale), 0, 2^bits-1) with IEEE division and
 * round-half-even. */
int rq_quantize(const void* w, rq_dtype w_dt, int64_t rows, int64_t cols, int group_size,
                int bits, uint32_t* w_q, void* scales, void* biases, void* stream);

/* mx.dequantize.  out[r, k] = T(T(code*scale) + bias) with T = sb_dt (MLX's
 * multiply-then-add in the scales dtype), then cast to out_dt. */
int rq_dequantize(const uint32_t* w_q, const void* scales, const void* biases, rq_dtype sb_dt,
                  int64_t rows, int64_t cols, int group_size, int bits, void* out,
                  rq_dtype out_dt, void* stream);

/* mx.quantized_matmul.  transpose=1: y[m, rows] = x[m, cols] . Ŵ^T;
 * transpose=0: y[m, cols] = x[m, rows] . Ŵ.  x_dt and sb_dt may differ
 * (MLX promotes both to a common type); accumulation is fp32; y in y_dt.
 * m <= 16 with transpose=1 runs the decode GEMV; larger m runs the MFMA GEMM.
 * Both multiply on bf16 MFMA operands.  The GEMV keeps every other step exact
 * (codes enter the MFMA as small integers, s and b are applied in fp32), and
 * at m <= 2 it multiplies fp32 or f16 x as two bf16 rows, bf16(x) and
 * bf16(x - bf16(x)), added at the end: y is then within ~1e-5 of the fp32
 * product.  At 2 < m <= 16 fp32 / f16 x is rounded to bf16 once, and the GEMM
 * also rounds each s*q + b to bf16: on N(0,1) fp32 x about 1.6e-3 (GEMV) and
 * 2.3e-3 (GEMM) Frobenius-relative from the fp32 product.  bf16 x loses
 * nothing to either.  At m >= 256 with 16-bit scales the GEMMs take bf16 and
 * fp32 x on the same kernels: fp32 x is rounded to bf16 as it is staged, so
 * its result equals that of bf16(x) with the same y_dt, bit for bit. */
int rq_qmm(const void* x, rq_dtype x_dt, const uint32_t* w_q, const void* scales,
           const void* biases, rq_dtype sb_dt, int64_t m, int64_t rows, int64_t cols,
           int group_size, int bits, int transpose, void* y, rq_dtype y_dt, void* stream);

/* rq_qmm(transpose=1) for prefill / training batches whose output tiles are
 * too few to fill the GPU over a long contraction (the same
 * mx.quantized_matmul at M = B*T, rwkv_metal/model/rwkv7_x070.py:131-144,
 * rwkv_metal/lora/finetune.py:115-117): the 64-wide-stage GEMM splits cols
 * into whole 8-group shares, writes fp32 partial tiles to `workspace` and a
 * second launch adds them in split order and rounds once into y_dt
 * (deterministic: the same bits on every call).  The split is chosen from a
 * cost model of this GPU; where it would not pay (or the 64-wide-stage
 * conditions of rq_qmm do not hold) this is exactly rq_qmm and the workspace
 * is not touched.  rq_qmm_splitk_workspace_bytes gives the bytes the call
 * needs for these sizes (0: none), or a negative rq error code (RQ_EINVAL,
 * rq_last_error set) for arguments rq_qmm would reject.  The workspace is
 * device memory, 16-byte aligned, needs no initialisation, and calls that
 * overlap in time need separate workspaces. */
int64_t rq_qmm_splitk_workspace_bytes(int64_t m, int64_t rows, int64_t cols, int group_size,
                                      int bits);
int rq_qmm_splitk(const void* x, rq_dtype x_dt, const uint32_t* w_q, const void* scales,
                  const void* biases, rq_dtype sb_dt, int64_t m, int64_t rows, int64_t cols,
                  int group_size, int bits, void* y, rq_dtype y_dt, void* workspace,
                  int64_t workspace_bytes, void* stream);

/* nn.QuantizedEmbedding lookup (upstream MLX; the "emb" target of
 * rwkv_metal/lora/finetune.py:42, looked up at rwkv_metal/model/rwkv7_x070.py:302):
 * out[i, :] = rq_dequantize of table row idx[i], for i < n, in one launch (the
 * gather is fused into the dequantization; no gathered copy of the packed
 * rows).  idx: int64[n] on the device; out: [n, cols] in out_dt.  The table is
 * [rows, cols].  An index outside [0, rows) yields a row of NaN and reads
 * nothing outside the table. */
int rq_embedding(const int64_t* idx, int64_t n, const uint32_t* w_q, const void* scales,
                 const void* biases, rq_dtype sb_dt, int64_t rows, int64_t cols, int group_size,
                 int bits, void* out, rq_dtype out_dt, void* stream);

/* rwkv-quant "sb6" tensors in the K3-interleaved layout RwkvqLinear holds
 * (rwkv_metal/lora/rwkvq_linear.py:96-110; layout stated at
 * rwkv_metal/lora/rwkvq_kernel.py:18-25).  The tensor is [rows, cols] in
 * blocks of gw_gs = 32 codes, nb = cols/32 blocks per row:
 *   qblk uint8[rows, nb*(16+4*xbits)]: per block 16 bytes (byte j = code j |
 *        code j+16 << 4), then for xbits >= 1 a uint32 bit plane (bit c = bit
 *        4 of code c), for xbits == 2 another (bit 5);
 *   qsqm uint8[rows, nb*2]: (qs uint8, qm int8) per block;
 *   ddm  float16[rows, (nb/gw_sb)*2]: (d, dm) per super-block of gw_sb blocks.
 * scale = f16(qs*d), min = f16(qm*dm), w = code*scale + min (fp32).
 * qblk and ddm 4-byte aligned, qsqm 2-byte aligned.
 *
 * rq_sb6_dequantize <- RwkvqLinear._dequant_w / the fused sb6 dequant kernel
 *   (rwkv_metal/lora/rwkvq_linear.py:131-135, rwkvq_kernel.py:86-124): dense
 *   out[rows, cols] in out_dt (fp32 as computed, or rounded to bf16/f16). */
int rq_sb6_dequantize(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm, int64_t rows,
                      int64_t cols, int gw_gs, int gw_sb, int xbits, void* out, rq_dtype out_dt,
                      void* stream);

/* rq_sb6_to_affine <- the one-time repack of RwkvqNativeLinear
 *   (rwkv_metal/lora/rwkvq_native.py:49-78, 103-113) into the MLX affine
 *   layout used by rq_qmm: w_q uint32[rows, nb*bits] with bits = 4 + xbits
 *   (codes bit for bit), scales = max(scale, 1e-8) and biases = min as fp32
 *   [rows, nb], group size 32.  w_q may be NULL (and then qblk too): only
 *   scales/biases are written (RwkvqHybridLinear._expand_scale_bias,
 *   rwkvq_hybrid.py:72-86).  Outputs 4-byte aligned. */
int rq_sb6_to_affine(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm, int64_t rows,
                     int64_t cols, int gw_gs, int gw_sb, int xbits, uint32_t* w_q, float* scales,
                     float* biases, void* stream);

/* The QLoRA layer's low-rank down-projection: z[m, rank] = x[m, k] . a[rank, k]^T,
 * bf16 in and out, fp32 accumulation; rank 16, 32, 48 or 64; k a multiple of 32;
 * x and a 16-byte aligned.  LoRALinear.__call__ (rwkv_metal/lora/lora.py:58-63)
 * computes z = x . A^T in the forward; MLX autograd computes u = dY . B in the
 * backward (a = B^T, [rank, out_features]).  Replaces those two mx.matmul nodes. */
int rq_lora_down(const void* x, int64_t m, int64_t k, const void* a, int64_t rank, void* z,
                 void* stream);

/* The QLoRA layer over a quantized base (LoRALinear.__call__,
 * rwkv_metal/lora/lora.py:58-63: base(x) + scale * (x A^T) B^T) with the
 * low-rank term fused into the GEMM's output stage:
 *   y = rq_qmm(x, ...) + scale * z . L^T
 * z: bf16 [m, rank]; lora (L): bf16 [n_out, rank], n_out = rows (transpose=1)
 * or cols (transpose=0).  Forward: z = x . lora_a^T, L = lora_b.  Backward dX
 * (the transpose=0 product of the QLoRA backward, finetune.py:141):
 * z = dY . lora_b, L = lora_a^T.  rank in {16, 32, 48, 64}; the term is
 * accumulated in fp32 with the GEMM and rounded once into y_dt.  Runs on the
 * 64-wide-stage GEMMs only (bf16 or fp32 x, m >= 256, 16-bit scales 16-byte aligned;
 * transpose=1: cols a multiple of 8 groups; transpose=0: rows % 64 == 0,
 * cols % 128 == 0, or cols % 160 == 0 with 4- or 8-bit codes); other
 * problems return RQ_EUNSUPPORTED and the caller
 * runs rq_qmm plus the term separately. */
int rq_qmm_lora(const void* x, rq_dtype x_dt, const uint32_t* w_q, const void* scales,
                const void* biases, rq_dtype sb_dt, int64_t m, int64_t rows, int64_t cols,
                int group_size, int bits, int transpose, const void* z, const void* lora,
                int64_t rank, float scale, void* y, rq_dtype y_dt, void* stream);

/* The QLoRA adapter gradients, the MLX autograd of LoRALinear.__call__
 * (rwkv_metal/lora/lora.py:58-63) through nn.value_and_grad
 * (rwkv_metal/lora/finetune.py:141), which the reference evaluates as two
 * mx.matmul nodes of its backward graph:
 *   da[rank, k] = scale * u^T . x     x [m, k], u = dY . B [m, rank]
 *   db[n, rank] = scale * dy^T . z    dy [m, n], z = x . A^T [m, rank]
 * in one launch: bf16 in and out, fp32 accumulation, one rounding of the
 * scaled sum.  Either product may be skipped with da = NULL (x and u are
 * then not read) or db = NULL.  rank 16, 32, 48 or 64; k and n multiples of
 * 8; x, u, dy and z 16-byte aligned.  m == 0 writes zero gradients.
 * Deterministic: the same inputs give the same bits.
 * The launch splits the m rows into chunks and reduces fp32 partial tiles in
 * `workspace`, rq_lora_grads_workspace_bytes(m, k, n, rank, da != NULL,
 * db != NULL) bytes (0 when one chunk per tile fills the GPU; workspace may
 * then be NULL), 16-byte aligned: 64 KiB of per-tile counters at fixed
 * offsets, then the partial tiles.  The workspace must be zero-filled before
 * its first use; every call leaves the counters at zero, so one workspace
 * serves any later problem that fits it.  Calls that run at the same time
 * need separate workspaces.  k/64 + n/64 is at most 16384.
 * rq_lora_grads_workspace_bytes returns a byte count (>= 0) or, for sizes
 * rq_lora_grads would reject, a negative rq error code (RQ_EINVAL) with
 * rq_last_error() set; check the sign before passing it to hipMalloc:
 *     int64_t nb = rq_lora_grads_workspace_bytes(m, k, n, rank, 1, 1);
 *     if (nb < 0) { fprintf(stderr, "%s\n", rq_last_error()); return nb; } */
int64_t rq_lora_grads_workspace_bytes(int64_t m, int64_t k, int64_t n, int64_t rank, int has_da,
                                      int has_db);
int rq_lora_grads(const void* x, const void* u, const void* dy, const void* z, int64_t m,
                  int64_t k, int64_t n, int64_t rank, float scale, void* da, void* db,
                  void* workspace, int64_t workspace_bytes, void* stream);

/* rq_lora_grads with fp32 x and dy (the reference's default activations:
 * fp32 residual stream, rwkv_metal/model/rwkv7_x070.py:51,189-194; the same
 * adapter gradients of rwkv_metal/lora/lora.py:58-63 under nn.value_and_grad,
 * rwkv_metal/lora/finetune.py:141).  u, z, da and db stay bf16.  x and dy are
 * rounded to bf16 as the kernel stages them (the products are bf16 MFMAs with
 * fp32 accumulation, as in rq_lora_grads); otherwise the same arguments,
 * workspace rules (rq_lora_grads_workspace_bytes) and determinism. */
int rq_lora_grads_f32(const float* x, const void* u, const float* dy, const void* z, int64_t m,
                      int64_t k, int64_t n, int64_t rank, float scale, void* da, void* db,
                      void* workspace, int64_t workspace_bytes, void* stream);

/* rq_lora_grads without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  It has no counterpart in the reference.
 * Same arguments, results (bit for bit) and kernels; the counters and
 * partial tiles live in a static device buffer of 8 MiB + 64 KiB per GPU,
 * held until the process ends, whose address is looked up at the first call
 * on each device, with the device of `stream` current.  Its counters are
 * cleared by a fill kernel on `stream` at the first call that is not being
 * captured into a graph (a call under capture puts the clear into the graph
 * ahead of its own launch until then).  The call allocates nothing.  Problems whose partial
 * tiles would not fit are rejected with RQ_EINVAL (the row split is capped
 * at 8 MiB, so that is k/64 + n/64 > 16384).  Every call on a GPU shares that
 * GPU's buffer: calls that overlap in time on one GPU (other streams, other
 * host threads) race and must be serialised by the caller. */
int rq_lora_grads_noalloc(const void* x, const void* u, const void* dy, const void* z, int64_t m,
                          int64_t k, int64_t n, int64_t rank, float scale, void* da, void* db,
                          void* stream);

/* The whole QLoRA layer product over a quantized base in ONE launch
 * (LoRALinear.__call__, rwkv_metal/lora/lora.py:58-63, and its dX under
 * nn.value_and_grad, rwkv_metal/lora/finetune.py:141): the down-projection
 * z = x . a^T is accumulated by the GEMM itself from the activation tiles it
 * already holds, then
 *   y = rq_qmm(x, ...) + scale * z . lora^T
 * and z is also stored to z_out [m, rank] bf16 (if not NULL) for the
 * backward.  Forward (transpose=1): a = lora_a [rank, cols], lora = lora_b
 * [rows, rank], z_out = x . lora_a^T.  dX (transpose=0): a = lora_b^T
 * [rank, rows], lora = lora_a^T [cols, rank], z_out = u = dY . lora_b.
 * z is rounded once to bf16 before the term, as rq_lora_down + rq_qmm_lora
 * do.  Large problems (with z_out given) take two launches instead: z as its
 * own pass, which reads x once, then the GEMM with the term in its output
 * stage -- exactly rq_lora_down + rq_qmm_lora on bf16(x); recomputing z in
 * every output column tile costs more there: outputs at least 4096 wide and
 * twice the contraction.  Covers rank 16 with 4- or 8-bit codes on the 64-wide-stage
 * GEMMs (the conditions of rq_qmm_lora); other problems return
 * RQ_EUNSUPPORTED (z_out may have been written) and the caller runs
 * rq_lora_down and rq_qmm_lora.  a, lora and z_out 16-byte aligned. */
int rq_qlora(const void* x, rq_dtype x_dt, const uint32_t* w_q, const void* scales,
             const void* biases, rq_dtype sb_dt, int64_t m, int64_t rows, int64_t cols,
             int group_size, int bits, int transpose, const void* a, const void* lora,
             int64_t rank, float scale, void* z_out, void* y, rq_dtype y_dt, void* stream);

/* The QLoRA layer's dX in ONE launch from the adapters as the layer stores
 * them (LoRALinear.lora_a [rank, cols] and lora_b [rows, rank] bf16,
 * rwkv_metal/lora/lora.py:55-56, differentiated as in
 * rwkv_metal/lora/finetune.py:141): u = dy . lora_b is accumulated by the
 * transposed GEMM from the dy tiles it already holds, then
 *   dx = rq_qmm(dy, ..., transpose=0) + scale * u . lora_a
 * and u is stored to u_out [m, rank] bf16 (if not NULL) for the adapter
 * gradients.  The same product as rq_qlora with transpose=0, a = lora_b^T
 * and lora = lora_a^T, bit for bit, without the two transposed copies
 * (also where it takes two launches: cols >= 4096 and >= 2 rows, u_out
 * given).  Covers what rq_qlora's dX covers (rank 16, 4- or 8-bit codes);
 * other problems return RQ_EUNSUPPORTED.  dy, w_q, lora_b and u_out 16-byte
 * aligned, lora_a 2-byte aligned. */
int rq_qlora_dx(const void* dy, rq_dtype dy_dt, const uint32_t* w_q, const void* scales,
                const void* biases, rq_dtype sb_dt, int64_t m, int64_t rows, int64_t cols,
                int group_size, int bits, const void* lora_a, const void* lora_b, int64_t rank,
                float scale, void* u_out, void* dx, rq_dtype dx_dt, void* stream);

/* Pack codes uint8[rows, cols] (values < 2^bits) into the MLX bitstream
 * w_q uint32[rows, cols*bits/32].  cols must be a multiple of 32. */
int rq_pack(const uint8_t* codes, int64_t rows, int64_t cols, int bits, uint32_t* w_q,
            void* stream);

/* Inverse of rq_pack: w_q -> codes uint8[rows, cols]. */
int rq_unpack(const uint32_t* w_q, int64_t rows, int64_t cols, int bits, uint8_t* codes,
              void* stream);

/* One transpose=True product of a grouped launch. */
typedef struct {
    const void* x;          /* [m, cols] in x_dt */
    const uint32_t* w_q;    /* [rows, cols*bits/32] */
    const void* scales;     /* [rows, cols/group_size] in sb_dt */
    const void* biases;
    void* y;                /* [m, rows] in y_dt */
    int64_t rows;
    int64_t cols;
} rq_problem;

/* Several independent decode GEMVs (m <= 16, transpose=True) sharing m, bits,
 * group_size and dtypes.  `problems` is a HOST array of n descriptors; they
 * are bucketed by cols and copied into kernel arguments, at most
 * RQ_MAX_GROUPED per launch: one launch per bucket per RQ_MAX_GROUPED
 * descriptors. */
#define RQ_MAX_GROUPED 48
int rq_qmm_grouped(const rq_problem* problems, int n, rq_dtype x_dt, rq_dtype sb_dt,
                   rq_dtype y_dt, int64_t m, int group_size, int bits, void* stream);

/* Planned grouped decode GEMV: the schedule of a fixed set of problems (the
 * projections one decode step runs, re-run every step with new activations
 * in the same buffers) is written once into caller-owned device memory, and
 * each run is ONE kernel launch however many problems there are.  Same
 * semantics as rq_qmm_grouped.  Like rq_qmm_grouped it has no single MLX
 * counterpart: it evaluates several independent mx.quantized_matmul
 * (transpose=True) nodes of one lazy graph (rwkv_metal/model/rwkv7_x070.py:142-144,
 * the 24-layer decode sweep of the benchmark).
 *
 * rq_grouped_plan_table_bytes: device bytes the table needs (or < 0 on error).
 * rq_grouped_plan_init: validates, orders the problems longest contraction
 *   first, uploads the table to `table` and SYNCHRONISES `stream` (the host
 *   staging copy does not outlive the call).  Returns RQ_EUNSUPPORTED for
 *   problems outside the planned kernels (scales must be 16-bit and
 *   16-byte aligned, cols % 512 == 0, and either m <= 4 with m*cols*2 bytes
 *   of activations within the LDS budget or 4 < m <= 16 with 4- or 8-bit
 *   codes); rq_qmm_grouped covers those.  Small sets (fewer than
 *   about 1024 blocks of 64 rows) run faster on rq_qmm_grouped, which splits
 *   them along K. 
 * rq_grouped_plan_run: one launch on `stream`.  The table and every pointer
 *   of the problems must stay valid for as long as the plan is run. */
typedef struct {
    int64_t opaque[8];
} rq_grouped_plan;
int64_t rq_grouped_plan_table_bytes(const rq_problem* problems, int n);
int rq_grouped_plan_init(const rq_problem* problems, int n, rq_dtype x_dt, rq_dtype sb_dt,
                         rq_dtype y_dt, int64_t m, int group_size, int bits, void* table,
                         int64_t table_bytes, rq_grouped_plan* plan, void* stream);
int rq_grouped_plan_run(const rq_grouped_plan* plan, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RWKVQ_H */
