// rq_launch.h -- host-side launchers, one per kernel family.  Arguments are
// validated by the C ABI layer (rq_abi.cpp) before any of these is called.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/rwkvq.h"

namespace rq {

hipError_t launch_quantize(const void* w, int w_dt, int64_t rows, int64_t cols, int gs, int bits,
                           uint32_t* wq, void* scales, void* biases, hipStream_t stream);

hipError_t launch_dequantize(const uint32_t* wq, const void* scales, const void* biases,
                             int sb_dt, int64_t rows, int64_t cols, int gs, int bits, void* out,
                             int out_dt, hipStream_t stream);

// Row gather + dequantize (embedding lookup): out[i] = dequantize(row idx[i]).
hipError_t launch_embedding(const int64_t* idx, int64_t n, const uint32_t* wq,
                            const void* scales, const void* biases, int sb_dt, int64_t rows,
                            int64_t cols, int gs, int bits, void* out, int out_dt,
                            hipStream_t stream);

// rwkv-quant sb6 (K3-interleaved) tensors: dense dequantize, and the repack
// into the MLX affine layout (bits = 4 + xbits, fp32 scales/biases, gs 32).
hipError_t launch_sb6_dequantize(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                                 int64_t rows, int64_t cols, int gw_sb, int xbits, void* out,
                                 int out_dt, hipStream_t stream);
hipError_t launch_sb6_to_affine(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                                int64_t rows, int64_t cols, int gw_sb, int xbits, uint32_t* wq,
                                float* scales, float* biases, hipStream_t stream);

hipError_t launch_pack(const uint8_t* codes, int64_t rows, int64_t cols, int bits, uint32_t* wq,
                       hipStream_t stream);

hipError_t launch_unpack(const uint32_t* wq, int64_t rows, int64_t cols, int bits,
                         uint8_t* codes, hipStream_t stream);

// Decode GEMV, transpose=True, 1 <= m <= 16, over n independent problems.
hipError_t launch_qmv(const rq_problem* problems, int n, int x_dt, int sb_dt, int y_dt,
                      int64_t m, int gs, int bits, hipStream_t stream);

// Streamed decode GEMV over a device-side schedule (rq_grouped_plan_*).
struct QmvTable {
    const rq_problem* descs;  // device: problem descriptors, longest K first
    const uint32_t* blocks;   // device: per block, problem << 16 | 64-row block of that problem
    int m, x_dt, y_dt;        // m: MFMA activation rows (2x the problems' m when xsplit)
    int xsplit;               // x runs as its hi/lo bf16 split (qmv_xsplit)
};
#ifndef RQ_QMV_XSPLIT
#define RQ_QMV_XSPLIT 1  // 0: round fp32/f16 activations to bf16 in the GEMV as well
#endif
// fp32 and f16 activations at m <= 2: the decode GEMV multiplies x as two
// bf16 rows, bf16(x) and bf16(x - bf16(x)) (16 significant bits: all of f16,
// fp32 to ~2^-17 relative), in MFMA rows that would otherwise be idle, and
// adds the two products before the output is stored.
inline bool qmv_xsplit(int x_dt, int64_t m) { return RQ_QMV_XSPLIT && x_dt != RQ_BF16 && m <= 2; }
inline int64_t qmv_rows(int x_dt, int64_t m) { return qmv_xsplit(x_dt, m) ? 2 * m : m; }
constexpr int kQmvLdsBudget = 64 * 1024;  // LDS bytes a GEMV block may stage
constexpr int kQmvRowsPerBlock = 64;      // rows of one streamed-GEMV block
// LDS bytes of a streamed-GEMV block for one problem shape.
size_t qmv_stream_lds(int64_t m, int64_t cols, int gs, int bits);
// Whether the streamed GEMV covers a problem (16-bit scales, cols % 512 == 0,
// 16-byte aligned scales/biases, staging within budget).
bool qmv_stream_covers(const rq_problem& p, int sb_dt, int64_t m, int gs, int bits);
hipError_t launch_qmv_table(const QmvTable& t, int blocks, int sb_dt, int gs, int bits,
                            size_t lds, hipStream_t stream);

// Split-K GEMM (transpose=1): fp32 partial tiles of `splits` shares of the
// contraction into part [splits][m][rows], then their in-order sum into y.
hipError_t launch_splitk_reduce(const float* part, int splits, int64_t m, int64_t rows, void* y,
                                int y_dt, hipStream_t stream);

// Low-rank term fused into the output stage of the 64-wide-stage GEMMs:
// y += scale * z . L^T with z [m, rank] and L [n_out, rank], both bf16,
// rank a multiple of 16 and at most 64.  A launcher given one returns
// hipErrorNotSupported when its problem does not run on those kernels.
struct LoraArgs {
    const void* z;
    const void* l;
    int rank;
    float scale;
    // In-kernel down-projection (rank 16): z = act . a^T is accumulated by the
    // GEMM's MFMA waves from the activation fragments they already hold (a:
    // [16, a_ld] bf16, a_ld the contraction length) instead of being read
    // from `z`, and written to z_out [m, 16] (if not NULL).
    const void* a = nullptr;
    void* z_out = nullptr;
    int64_t a_ld = 0;
    // The transposed GEMM's down-projection from the adapters as a LoRA
    // layer stores them (transpose=0, rank 16): `a` is then B [a_ld, 16]
    // (element (j, c) of a at a[c * 16 + j]) and `l` is A [16, l_ld]
    // (element (n, j) of L at l[j * l_ld + n]), so that dX needs no
    // transposed copies of the adapters.
    bool stored = false;
    int64_t l_ld = 0;
};

// Low-rank down-projection z[m, rank] = x[m, k] . a[rank, k]^T, bf16 (rank
// 16, 32, 48 or 64; k a multiple of 32).  a_t: the adapter is given as
// a^T [k, rank] (row-major, 16-byte aligned) instead.  x_f32: x is fp32
// (rounded to bf16 as it is read; z is then that of bf16(x)).
hipError_t launch_lora_down(const void* x, int64_t m, int64_t k, const void* a, int rank, void* z,
                            hipStream_t stream, bool a_t = false, bool x_f32 = false);

// QLoRA adapter gradients dA[rank, k] = scale * u^T x and dB[n, rank] =
// scale * dY^T z in one launch (bf16 in and out, fp32 accumulation).  The
// plan splits the m rows into `splits` chunks per 64-column tile; with more
// than one, the launch needs a work buffer of kLoraGradCounterBytes of
// per-tile counters (at fixed offsets, so that a counter slot never holds
// anything else: zero before the first use, left zero by every launch,
// whatever problem used the buffer last) followed by `partial_bytes` of fp32
// partial tiles.
constexpr int kLoraGradTargetBlocks = 512;           // ~2 jobs per CU
constexpr int64_t kLoraGradPartialCap = 8ll << 20;   // fp32 partial bytes at most
constexpr int kLoraGradMaxTiles = 16384;             // k/64 + n/64 at most
constexpr size_t kLoraGradCounterBytes = (size_t)kLoraGradMaxTiles * 4;
struct LoraGradPlan {
    int tiles_a, tiles_b, splits;
    int64_t mchunk;         // rows per chunk (a multiple of 64)
    size_t partial_bytes;   // 0 when splits == 1
    size_t work_bytes;      // counters + partials; 0 when splits == 1
};
LoraGradPlan lora_grads_plan(int64_t m, int64_t k, int64_t n, int rank, bool has_a, bool has_b);
// The no-allocation form's work buffer: a static device array of
// kLoraScratchBytes per GPU.  lora_scratch gives its address on the current
// device (looked up, and its counters cleared on `stream`, at the first call
// on that device).
constexpr size_t kLoraScratchBytes = kLoraGradCounterBytes + (size_t)kLoraGradPartialCap;
hipError_t lora_scratch(void** out, hipStream_t stream);
// xdy_f32: x and dy are fp32 (u, z, da, db bf16).
hipError_t launch_lora_grads(const void* x, const void* u, const void* dy, const void* z,
                             int64_t m, int64_t k, int64_t n, int rank, float scale, void* da,
                             void* db, const LoraGradPlan& p, void* work, hipStream_t stream,
                             bool xdy_f32 = false);

// MFMA GEMM, transpose=True: y[m, rows] = x[m, cols] . W^T.
hipError_t launch_qmm_t(const void* x, int x_dt, const uint32_t* wq, const void* scales,
                        const void* biases, int sb_dt, int64_t m, int64_t rows, int64_t cols,
                        int gs, int bits, void* y, int y_dt, hipStream_t stream,
                        const LoraArgs* lora = nullptr);

// MFMA GEMM, transpose=False: y[m, cols] = x[m, rows] . W.
hipError_t launch_qmm_n(const void* x, int x_dt, const uint32_t* wq, const void* scales,
                        const void* biases, int sb_dt, int64_t m, int64_t rows, int64_t cols,
                        int gs, int bits, void* y, int y_dt, hipStream_t stream,
                        const LoraArgs* lora = nullptr);

}  // namespace rq
