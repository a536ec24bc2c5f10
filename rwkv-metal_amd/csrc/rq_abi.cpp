// rq_abi.cpp -- the extern "C" boundary of librwkvq_hip.so (include/rwkvq.h).
//
// Validates arguments the way MLX's quantization ops do (bits, group size,
// shapes and dtypes), checks alignment, then dispatches to the kernel
// launchers.  Every failure returns a negative code and leaves a message in a
// thread-local buffer read by rq_last_error().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/rwkvq.h"
#include "rq_launch.h"

namespace rq {

#define RQ_DECLARE_BITS(B)                                                                     \
    hipError_t launch_qmv_b##B(const rq_problem*, int, int, int, int, int64_t, int,             \
                               hipStream_t);                                                    \
    hipError_t launch_qmm_t_b##B(const void*, int, const uint32_t*, const void*, const void*,    \
                                 int, int64_t, int64_t, int64_t, int, void*, int, hipStream_t,  \
                                 const LoraArgs*);                                              \
    hipError_t launch_qmm_n_b##B(const void*, int, const uint32_t*, const void*, const void*,    \
                                 int, int64_t, int64_t, int64_t, int, void*, int, hipStream_t,  \
                                 const LoraArgs*);                                              \
    hipError_t launch_qmm_t_splitk_b##B(const void*, int, const uint32_t*, const void*,          \
                                        const void*, int, int64_t, int64_t, int64_t, int, int,   \
                                        int, float*, hipStream_t);
#define RQ_DECLARE_TABLE(B)                                                                    \
    hipError_t launch_qmv_table_b##B(const QmvTable&, int, int, int, size_t, hipStream_t);
RQ_DECLARE_TABLE(2)
RQ_DECLARE_TABLE(3)
RQ_DECLARE_TABLE(4)
RQ_DECLARE_TABLE(5)
RQ_DECLARE_TABLE(6)
RQ_DECLARE_TABLE(8)

hipError_t launch_qmv_table(const QmvTable& t, int blocks, int sb_dt, int gs, int bits,
                            size_t lds, hipStream_t stream) {
    switch (bits) {
        case 2: return launch_qmv_table_b2(t, blocks, sb_dt, gs, lds, stream);
        case 3: return launch_qmv_table_b3(t, blocks, sb_dt, gs, lds, stream);
        case 4: return launch_qmv_table_b4(t, blocks, sb_dt, gs, lds, stream);
        case 5: return launch_qmv_table_b5(t, blocks, sb_dt, gs, lds, stream);
        case 6: return launch_qmv_table_b6(t, blocks, sb_dt, gs, lds, stream);
        case 8: return launch_qmv_table_b8(t, blocks, sb_dt, gs, lds, stream);
        default: return hipErrorInvalidValue;
    }
}

RQ_DECLARE_BITS(2)
RQ_DECLARE_BITS(3)
RQ_DECLARE_BITS(4)
RQ_DECLARE_BITS(5)
RQ_DECLARE_BITS(6)
RQ_DECLARE_BITS(8)

hipError_t launch_qmv(const rq_problem* problems, int n, int x_dt, int sb_dt, int y_dt,
                      int64_t m, int gs, int bits, hipStream_t stream) {
    switch (bits) {
        case 2: return launch_qmv_b2(problems, n, x_dt, sb_dt, y_dt, m, gs, stream);
        case 3: return launch_qmv_b3(problems, n, x_dt, sb_dt, y_dt, m, gs, stream);
        case 4: return launch_qmv_b4(problems, n, x_dt, sb_dt, y_dt, m, gs, stream);
        case 5: return launch_qmv_b5(problems, n, x_dt, sb_dt, y_dt, m, gs, stream);
        case 6: return launch_qmv_b6(problems, n, x_dt, sb_dt, y_dt, m, gs, stream);
        case 8: return launch_qmv_b8(problems, n, x_dt, sb_dt, y_dt, m, gs, stream);
        default: return hipErrorInvalidValue;
    }
}

#define RQ_QMM_SWITCH(FN)                                                                      \
    switch (bits) {                                                                            \
        case 2: return FN##2(x, x_dt, wq, scales, biases, sb_dt, m, rows, cols, gs, y, y_dt, stream, lora); \
        case 3: return FN##3(x, x_dt, wq, scales, biases, sb_dt, m, rows, cols, gs, y, y_dt, stream, lora); \
        case 4: return FN##4(x, x_dt, wq, scales, biases, sb_dt, m, rows, cols, gs, y, y_dt, stream, lora); \
        case 5: return FN##5(x, x_dt, wq, scales, biases, sb_dt, m, rows, cols, gs, y, y_dt, stream, lora); \
        case 6: return FN##6(x, x_dt, wq, scales, biases, sb_dt, m, rows, cols, gs, y, y_dt, stream, lora); \
        case 8: return FN##8(x, x_dt, wq, scales, biases, sb_dt, m, rows, cols, gs, y, y_dt, stream, lora); \
        default: return hipErrorInvalidValue;                                                  \
    }

static hipError_t launch_qmm(int transpose, const void* x, int x_dt, const uint32_t* wq,
                             const void* scales, const void* biases, int sb_dt, int64_t m,
                             int64_t rows, int64_t cols, int gs, int bits, void* y, int y_dt,
                             hipStream_t stream, const LoraArgs* lora = nullptr) {
    if (transpose) {
        RQ_QMM_SWITCH(launch_qmm_t_b)
    } else {
        RQ_QMM_SWITCH(launch_qmm_n_b)
    }
}

}  // namespace rq

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_err[0] = '\0';
    return RQ_OK;
}

bool valid_bits(int b) { return b == 2 || b == 3 || b == 4 || b == 5 || b == 6 || b == 8; }
bool valid_gs(int g) { return g == 32 || g == 64 || g == 128; }
bool valid_dt(int d) { return d == RQ_BF16 || d == RQ_F16 || d == RQ_F32; }
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_common(int64_t rows, int64_t cols, int gs, int bits) {
    if (!valid_bits(bits)) return fail(RQ_EINVAL, "bits must be one of 2,3,4,5,6,8 (got %d)", bits);
    if (!valid_gs(gs)) return fail(RQ_EINVAL, "group_size must be 32, 64 or 128 (got %d)", gs);
    if (rows < 0 || cols < 0) return fail(RQ_EINVAL, "negative size (rows=%lld cols=%lld)",
                                          (long long)rows, (long long)cols);
    if (cols % gs != 0)
        return fail(RQ_EINVAL, "the last dimension (%lld) must be divisible by group_size %d",
                    (long long)cols, gs);
    return RQ_OK;
}

int launch_status(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(RQ_ELAUNCH, "%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return ok();
}

}  // namespace

extern "C" {

int rq_abi_version(void) { return RWKVQ_ABI_VERSION; }

const char* rq_last_error(void) { return g_err; }

int rq_quantize(const void* w, rq_dtype w_dt, int64_t rows, int64_t cols, int group_size, int bits,
                uint32_t* w_q, void* scales, void* biases, void* stream) {
    if (int rc = check_common(rows, cols, group_size, bits)) return rc;
    if (!valid_dt(w_dt)) return fail(RQ_EINVAL, "unsupported weight dtype %d", (int)w_dt);
    if (rows * cols == 0) return ok();
    if (!w || !w_q || !scales || !biases) return fail(RQ_EINVAL, "rq_quantize: NULL pointer");
    if (!aligned16(w) || !aligned16(w_q)) return fail(RQ_EALIGN, "rq_quantize: w and w_q must be 16-byte aligned");
    return launch_status(rq::launch_quantize(w, w_dt, rows, cols, group_size, bits, w_q, scales,
                                             biases, (hipStream_t)stream),
                         "rq_quantize");
}

int rq_dequantize(const uint32_t* w_q, const void* scales, const void* biases, rq_dtype sb_dt,
                  int64_t rows, int64_t cols, int group_size, int bits, void* out,
                  rq_dtype out_dt, void* stream) {
    if (int rc = check_common(rows, cols, group_size, bits)) return rc;
    if (!valid_dt(sb_dt) || !valid_dt(out_dt)) return fail(RQ_EINVAL, "unsupported dtype");
    if (rows * cols == 0) return ok();
    if (!w_q || !scales || !biases || !out) return fail(RQ_EINVAL, "rq_dequantize: NULL pointer");
    if (!aligned16(w_q) || !aligned16(out)) return fail(RQ_EALIGN, "rq_dequantize: w_q and out must be 16-byte aligned");
    return launch_status(rq::launch_dequantize(w_q, scales, biases, sb_dt, rows, cols, group_size,
                                               bits, out, out_dt, (hipStream_t)stream),
                         "rq_dequantize");
}

int rq_embedding(const int64_t* idx, int64_t n, const uint32_t* w_q, const void* scales,
                 const void* biases, rq_dtype sb_dt, int64_t rows, int64_t cols, int group_size,
                 int bits, void* out, rq_dtype out_dt, void* stream) {
    if (int rc = check_common(rows, cols, group_size, bits)) return rc;
    if (n < 0) return fail(RQ_EINVAL, "rq_embedding: negative n");
    if (!valid_dt(sb_dt) || !valid_dt(out_dt)) return fail(RQ_EINVAL, "unsupported dtype");
    if (n * cols == 0) return ok();
    if (!idx || !w_q || !scales || !biases || !out) return fail(RQ_EINVAL, "rq_embedding: NULL pointer");
    if (!aligned16(w_q) || !aligned16(out)) return fail(RQ_EALIGN, "rq_embedding: w_q and out must be 16-byte aligned");
    return launch_status(rq::launch_embedding(idx, n, w_q, scales, biases, sb_dt, rows, cols,
                                              group_size, bits, out, out_dt, (hipStream_t)stream),
                         "rq_embedding");
}

// qblk is read only when codes are decoded (need_codes).
static int check_sb6(const char* what, const uint8_t* qblk, const uint8_t* qsqm,
                     const uint16_t* ddm, int64_t rows, int64_t cols, int gw_gs, int gw_sb,
                     int xbits, bool need_codes) {
    if (rows < 0 || cols < 0) return fail(RQ_EINVAL, "%s: negative size", what);
    if (gw_gs != 32) return fail(RQ_EINVAL, "%s: sb6 blocks are 32 codes (gw_gs=%d)", what, gw_gs);
    if (cols % 32) return fail(RQ_EINVAL, "%s: cols %lld is not a multiple of 32", what, (long long)cols);
    if (xbits < 0 || xbits > 2) return fail(RQ_EINVAL, "%s: xbits must be 0, 1 or 2 (got %d)", what, xbits);
    if (gw_sb <= 0 || (cols / 32) % gw_sb)
        return fail(RQ_EINVAL, "%s: gw_sb=%d does not divide the %lld blocks per row", what, gw_sb,
                    (long long)(cols / 32));
    if (rows * cols && ((need_codes && !qblk) || !qsqm || !ddm))
        return fail(RQ_EINVAL, "%s: NULL pointer", what);
    if (((uintptr_t)qblk & 3) || ((uintptr_t)qsqm & 1) || ((uintptr_t)ddm & 3))
        return fail(RQ_EALIGN, "%s: qblk and ddm must be 4-byte aligned, qsqm 2-byte aligned", what);
    return RQ_OK;
}

int rq_sb6_dequantize(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm, int64_t rows,
                      int64_t cols, int gw_gs, int gw_sb, int xbits, void* out, rq_dtype out_dt,
                      void* stream) {
    if (int rc = check_sb6("rq_sb6_dequantize", qblk, qsqm, ddm, rows, cols, gw_gs, gw_sb, xbits,
                           true))
        return rc;
    if (!valid_dt(out_dt)) return fail(RQ_EINVAL, "unsupported dtype");
    if (rows * cols == 0) return ok();
    if (!out) return fail(RQ_EINVAL, "rq_sb6_dequantize: NULL output");
    if (!aligned16(out)) return fail(RQ_EALIGN, "rq_sb6_dequantize: out must be 16-byte aligned");
    return launch_status(rq::launch_sb6_dequantize(qblk, qsqm, ddm, rows, cols, gw_sb, xbits, out,
                                                   out_dt, (hipStream_t)stream),
                         "rq_sb6_dequantize");
}

int rq_sb6_to_affine(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm, int64_t rows,
                     int64_t cols, int gw_gs, int gw_sb, int xbits, uint32_t* w_q, float* scales,
                     float* biases, void* stream) {
    if (int rc = check_sb6("rq_sb6_to_affine", qblk, qsqm, ddm, rows, cols, gw_gs, gw_sb, xbits,
                           w_q != nullptr))
        return rc;
    if (rows * cols == 0) return ok();
    if (!scales || !biases) return fail(RQ_EINVAL, "rq_sb6_to_affine: NULL scales/biases");
    if (((uintptr_t)w_q | (uintptr_t)scales | (uintptr_t)biases) & 3)
        return fail(RQ_EALIGN, "rq_sb6_to_affine: outputs must be 4-byte aligned");
    return launch_status(rq::launch_sb6_to_affine(qblk, qsqm, ddm, rows, cols, gw_sb, xbits, w_q,
                                                  scales, biases, (hipStream_t)stream),
                         "rq_sb6_to_affine");
}

int rq_pack(const uint8_t* codes, int64_t rows, int64_t cols, int bits, uint32_t* w_q,
            void* stream) {
    if (int rc = check_common(rows, cols, 32, bits)) return rc;
    if (rows * cols == 0) return ok();
    if (!codes || !w_q) return fail(RQ_EINVAL, "rq_pack: NULL pointer");
    if (!aligned16(codes) || !aligned16(w_q)) return fail(RQ_EALIGN, "rq_pack: pointers must be 16-byte aligned");
    return launch_status(rq::launch_pack(codes, rows, cols, bits, w_q, (hipStream_t)stream), "rq_pack");
}

int rq_unpack(const uint32_t* w_q, int64_t rows, int64_t cols, int bits, uint8_t* codes,
              void* stream) {
    if (int rc = check_common(rows, cols, 32, bits)) return rc;
    if (rows * cols == 0) return ok();
    if (!codes || !w_q) return fail(RQ_EINVAL, "rq_unpack: NULL pointer");
    if (!aligned16(codes) || !aligned16(w_q)) return fail(RQ_EALIGN, "rq_unpack: pointers must be 16-byte aligned");
    return launch_status(rq::launch_unpack(w_q, rows, cols, bits, codes, (hipStream_t)stream), "rq_unpack");
}

// Split-K plan for the 64-wide-stage transpose=1 GEMM.  A cost model over
// measured per-stage times of one MI355X (1.13 us per 64-wide stage of a
// 256-row tile, 0.875 us of a 128-row one, 0.43 us of a 64 x 96 one; 256
// CUs, one block each) and the partial tiles' traffic (written and read once
// at ~5 TB/s, plus ~3 us for the reduction launch): the split that beats the
// unsplit launcher's own tile choice by 10 % or more, else none.  Splitting
// pays where few tiles meet a long contraction (config 3's [2560, 10240] at
// M = 512 / 2048), not where the partials cost as much as the work.
struct SplitKPlan {
    int bm = 256, splits = 1;
};

static bool splitk_applies(rq_dtype x_dt, rq_dtype sb_dt, int64_t m, int64_t cols, int gs,
                           const void* x, const void* scales, const void* biases) {
    return m >= 256 && (x_dt == RQ_BF16 || x_dt == RQ_F32) && sb_dt != RQ_F32 && cols % 64 == 0 &&
           (cols / gs) % 8 == 0 &&
           (((uintptr_t)x | (uintptr_t)scales | (uintptr_t)biases) & 15) == 0;
}

static SplitKPlan splitk_plan(int64_t m, int64_t rows, int64_t cols, int gs, int bits) {
    const int P = gs / 8;                            // 64-wide stages per 8-group period
    const int64_t nper = cols / (8 * (int64_t)gs);   // periods of the contraction
    const int bn = (bits == 4 && rows % 160 == 0) ? 160 : 128;
    const int64_t tn = (rows + bn - 1) / bn;
    auto cost = [&](int bm, int64_t tiles, int64_t splits, double stage_us) {
        const int64_t rounds = (tiles * splits + 255) / 256;
        const int64_t periods = (nper + splits - 1) / splits;
        double t = (double)rounds * (double)(periods * P) * stage_us;
        if (splits > 1) t += 2.0 * (double)splits * (double)(m * rows) * 4.0 / 5e6 + 3.0;
        (void)bm;
        return t;
    };
    // the unsplit launcher's choice (launch_qmm_t_b*)
    const int64_t t256 = ((m + 255) / 256) * tn, t128 = ((m + 127) / 128) * tn;
    double plain;
    if (t256 >= 200) plain = cost(256, t256, 1, 1.13);
    else if (bits == 4 && t128 < 128) plain = cost(64, ((m + 63) / 64) * ((rows + 95) / 96), 1, 0.43);
    else plain = cost(128, t128, 1, 0.875);
    SplitKPlan best;
    double bt = 0.9 * plain;
    for (int bm : {256, 128}) {
        const int64_t tiles = bm == 256 ? t256 : t128;
        const double stage_us = bm == 256 ? 1.13 : 0.875;
        for (int64_t s = 2; s <= nper && s <= 32 && tiles * s <= 1024; ++s) {
            const double t = cost(bm, tiles, s, stage_us);
            if (t < bt) {
                bt = t;
                best.bm = bm;
                best.splits = (int)s;
            }
        }
    }
    return best;
}

int64_t rq_qmm_splitk_workspace_bytes(int64_t m, int64_t rows, int64_t cols, int group_size,
                                      int bits) {
    if (int rc = check_common(rows, cols, group_size, bits)) return rc;
    if (m < 0) return fail(RQ_EINVAL, "rq_qmm_splitk_workspace_bytes: negative m");
    if (m < 256 || cols % 64 || (cols / group_size) % 8) return 0;
    const SplitKPlan p = splitk_plan(m, rows, cols, group_size, bits);
    return p.splits > 1 ? (int64_t)p.splits * m * rows * 4 : 0;
}

int rq_qmm_splitk(const void* x, rq_dtype x_dt, const uint32_t* w_q, const void* scales,
                  const void* biases, rq_dtype sb_dt, int64_t m, int64_t rows, int64_t cols,
                  int group_size, int bits, void* y, rq_dtype y_dt, void* workspace,
                  int64_t workspace_bytes, void* stream) {
    if (int rc = check_common(rows, cols, group_size, bits)) return rc;
    if (!valid_dt(x_dt) || !valid_dt(sb_dt) || !valid_dt(y_dt)) return fail(RQ_EINVAL, "unsupported dtype");
    if (m < 0) return fail(RQ_EINVAL, "negative m");
    SplitKPlan p;
    if (splitk_applies(x_dt, sb_dt, m, cols, group_size, x, scales, biases))
        p = splitk_plan(m, rows, cols, group_size, bits);
    if (p.splits <= 1)  // not worth splitting (or not the 64-wide-stage GEMM): rq_qmm itself
        return rq_qmm(x, x_dt, w_q, scales, biases, sb_dt, m, rows, cols, group_size, bits, 1, y,
                      y_dt, stream);
    if (rows == 0) return ok();
    if (!y || !x || !w_q || !scales || !biases) return fail(RQ_EINVAL, "rq_qmm_splitk: NULL pointer");
    if (!aligned16(x) || !aligned16(w_q))
        return fail(RQ_EALIGN, "rq_qmm_splitk: x and w_q must be 16-byte aligned");
    const int64_t need = (int64_t)p.splits * m * rows * 4;
    if (!workspace || workspace_bytes < need)
        return fail(RQ_EINVAL, "rq_qmm_splitk: workspace has %lld bytes, needs %lld",
                    (long long)workspace_bytes, (long long)need);
    if (!aligned16(workspace)) return fail(RQ_EALIGN, "rq_qmm_splitk: workspace must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    float* part = (float*)workspace;
    hipError_t e;
    switch (bits) {
#define RQ_SKB(B)                                                                                 \
    case B:                                                                                      \
        e = rq::launch_qmm_t_splitk_b##B(x, x_dt, w_q, scales, biases, sb_dt, m, rows, cols,       \
                                         group_size, p.bm, p.splits, part, s);                  \
        break;
        RQ_SKB(2) RQ_SKB(3) RQ_SKB(4) RQ_SKB(5) RQ_SKB(6) RQ_SKB(8)
#undef RQ_SKB
        default: e = hipErrorInvalidValue;
    }
    if (e != hipSuccess) return launch_status(e, "rq_qmm_splitk");
    return launch_status(rq::launch_splitk_reduce(part, p.splits, m, rows, y, y_dt, s),
                         "rq_qmm_splitk");
}

int rq_qmm(const void* x, rq_dtype x_dt, const uint32_t* w_q, const void* scales,
           const void* biases, rq_dtype sb_dt, int64_t m, int64_t rows, int64_t cols,
           int group_size, int bits, int transpose, void* y, rq_dtype y_dt, void* stream) {
    if (int rc = check_common(rows, cols, group_size, bits)) return rc;
    if (!valid_dt(x_dt) || !valid_dt(sb_dt) || !valid_dt(y_dt)) return fail(RQ_EINVAL, "unsupported dtype");
    if (m < 0) return fail(RQ_EINVAL, "negative m");
    const int64_t n_out = transpose ? rows : cols;
    if (m == 0 || n_out == 0) return ok();
    if (!y) return fail(RQ_EINVAL, "rq_qmm: NULL output");
    const int64_t n_in = transpose ? cols : rows;
    if (n_in == 0) return fail(RQ_EINVAL, "rq_qmm: empty contraction with a non-empty output is not supported");
    if (!x || !w_q || !scales || !biases) return fail(RQ_EINVAL, "rq_qmm: NULL pointer");
    if (!aligned16(x) || !aligned16(w_q)) return fail(RQ_EALIGN, "rq_qmm: x and w_q must be 16-byte aligned");
    hipError_t e;
    if (transpose && m <= 16) {
        rq_problem p = {x, w_q, scales, biases, y, rows, cols};
        e = rq::launch_qmv(&p, 1, x_dt, sb_dt, y_dt, m, group_size, bits, (hipStream_t)stream);
    } else {
        e = rq::launch_qmm(transpose, x, x_dt, w_q, scales, biases, sb_dt, m, rows, cols,
                           group_size, bits, y, y_dt, (hipStream_t)stream);
    }
    return launch_status(e, "rq_qmm");
}

int rq_lora_down(const void* x, int64_t m, int64_t k, const void* a, int64_t rank, void* z,
                 void* stream) {
    if (m < 0 || k < 0) return fail(RQ_EINVAL, "rq_lora_down: negative size");
    if (rank < 16 || rank > 64 || rank % 16)
        return fail(RQ_EINVAL, "rq_lora_down: rank must be 16, 32, 48 or 64 (got %lld)", (long long)rank);
    if (k % 32) return fail(RQ_EINVAL, "rq_lora_down: k must be a multiple of 32 (got %lld)", (long long)k);
    if (m == 0) return ok();
    if (k == 0) return fail(RQ_EINVAL, "rq_lora_down: empty contraction is not supported");
    if (!x || !a || !z) return fail(RQ_EINVAL, "rq_lora_down: NULL pointer");
    if (!aligned16(x) || !aligned16(a)) return fail(RQ_EALIGN, "rq_lora_down: x and a must be 16-byte aligned");
    return launch_status(rq::launch_lora_down(x, m, k, a, (int)rank, z, (hipStream_t)stream),
                         "rq_lora_down");
}

static int check_lora_grads(const char* what, const void* x, const void* u, const void* dy,
                            const void* z, int64_t m, int64_t k, int64_t n, int64_t rank,
                            const void* da, const void* db) {
    if (m < 0 || k < 0 || n < 0) return fail(RQ_EINVAL, "%s: negative size", what);
    if (rank < 16 || rank > 64 || rank % 16)
        return fail(RQ_EINVAL, "%s: rank must be 16, 32, 48 or 64 (got %lld)", what, (long long)rank);
    if (da && k % 8) return fail(RQ_EINVAL, "%s: k must be a multiple of 8 (got %lld)", what, (long long)k);
    if (db && n % 8) return fail(RQ_EINVAL, "%s: n must be a multiple of 8 (got %lld)", what, (long long)n);
    if (m > 0 && ((da && k > 0 && (!x || !u)) || (db && n > 0 && (!dy || !z))))
        return fail(RQ_EINVAL, "%s: NULL operand", what);
    if ((da && (!aligned16(x) || !aligned16(u))) || (db && (!aligned16(dy) || !aligned16(z))))
        return fail(RQ_EALIGN, "%s: x, u, dy and z must be 16-byte aligned", what);
    return RQ_OK;
}

int64_t rq_lora_grads_workspace_bytes(int64_t m, int64_t k, int64_t n, int64_t rank, int has_da,
                                      int has_db) {
    if (m < 0 || k < 0 || n < 0 || rank < 16 || rank > 64 || rank % 16)
        return fail(RQ_EINVAL, "rq_lora_grads_workspace_bytes: bad sizes");
    const rq::LoraGradPlan p = rq::lora_grads_plan(m, k, n, (int)rank, has_da != 0, has_db != 0);
    if (p.tiles_a + p.tiles_b > rq::kLoraGradMaxTiles)
        return fail(RQ_EINVAL, "rq_lora_grads_workspace_bytes: k/64 + n/64 exceeds %d",
                    rq::kLoraGradMaxTiles);
    return (int64_t)p.work_bytes;
}

static int lora_grads_common(const char* what, const void* x, const void* u, const void* dy,
                             const void* z, int64_t m, int64_t k, int64_t n, int64_t rank,
                             float scale, void* da, void* db, void* workspace,
                             int64_t workspace_bytes, void* stream, bool xdy_f32) {
    if (int rc = check_lora_grads(what, x, u, dy, z, m, k, n, rank, da, db)) return rc;
    hipStream_t s = (hipStream_t)stream;
    // m == 0 runs too: every job then stores a zero tile (no memset, so the
    // call may be captured in a HIP graph)
    const rq::LoraGradPlan p =
        rq::lora_grads_plan(m, k, n, (int)rank, da != nullptr, db != nullptr);
    if (p.tiles_a + p.tiles_b > rq::kLoraGradMaxTiles)
        return fail(RQ_EINVAL, "%s: k/64 + n/64 exceeds %d", what, rq::kLoraGradMaxTiles);
    const int64_t need = (int64_t)p.work_bytes;
    if (need > 0) {
        if (!workspace || workspace_bytes < need)
            return fail(RQ_EINVAL, "%s: workspace has %lld bytes, needs %lld", what,
                        (long long)workspace_bytes, (long long)need);
        if (!aligned16(workspace))
            return fail(RQ_EALIGN, "%s: workspace must be 16-byte aligned", what);
    }
    return launch_status(rq::launch_lora_grads(x, u, dy, z, m, k, n, (int)rank, scale, da, db, p,
                                               workspace, s, xdy_f32),
                         what);
}

int rq_lora_grads(const void* x, const void* u, const void* dy, const void* z, int64_t m,
                  int64_t k, int64_t n, int64_t rank, float scale, void* da, void* db,
                  void* workspace, int64_t workspace_bytes, void* stream) {
    return lora_grads_common("rq_lora_grads", x, u, dy, z, m, k, n, rank, scale, da, db,
                             workspace, workspace_bytes, stream, false);
}

int rq_lora_grads_f32(const float* x, const void* u, const float* dy, const void* z, int64_t m,
                      int64_t k, int64_t n, int64_t rank, float scale, void* da, void* db,
                      void* workspace, int64_t workspace_bytes, void* stream) {
    return lora_grads_common("rq_lora_grads_f32", x, u, dy, z, m, k, n, rank, scale, da, db,
                             workspace, workspace_bytes, stream, true);
}

int rq_lora_grads_noalloc(const void* x, const void* u, const void* dy, const void* z, int64_t m,
                          int64_t k, int64_t n, int64_t rank, float scale, void* da, void* db,
                          void* stream) {
    if (int rc = check_lora_grads("rq_lora_grads_noalloc", x, u, dy, z, m, k, n, rank, da, db))
        return rc;
    const rq::LoraGradPlan p =
        rq::lora_grads_plan(m, k, n, (int)rank, da != nullptr, db != nullptr);
    if (p.tiles_a + p.tiles_b > rq::kLoraGradMaxTiles)
        return fail(RQ_EINVAL, "rq_lora_grads_noalloc: k/64 + n/64 exceeds %d",
                    rq::kLoraGradMaxTiles);
    if (p.work_bytes > rq::kLoraScratchBytes)
        return fail(RQ_EINVAL, "rq_lora_grads_noalloc: needs %lld bytes of scratch, the static "
                    "buffer holds %lld", (long long)p.work_bytes, (long long)rq::kLoraScratchBytes);
    hipStream_t s = (hipStream_t)stream;
    void* work = nullptr;
    if (p.work_bytes > 0) {
        const hipError_t e = rq::lora_scratch(&work, s);
        if (e != hipSuccess)
            return fail(RQ_ELAUNCH, "rq_lora_grads_noalloc: static scratch unavailable: %s",
                        hipGetErrorString(e));
    }
    return launch_status(rq::launch_lora_grads(x, u, dy, z, m, k, n, (int)rank, scale, da, db, p,
                                               work, s),
                         "rq_lora_grads_noalloc");
}

int rq_qmm_lora(const void* x, rq_dtype x_dt, const uint32_t* w_q, const void* scales,
                const void* biases, rq_dtype sb_dt, int64_t m, int64_t rows, int64_t cols,
                int group_size, int bits, int transpose, const void* z, const void* lora,
                int64_t rank, float scale, void* y, rq_dtype y_dt, void* stream) {
    if (int rc = check_common(rows, cols, group_size, bits)) return rc;
    if (!valid_dt(x_dt) || !valid_dt(sb_dt) || !valid_dt(y_dt)) return fail(RQ_EINVAL, "unsupported dtype");
    if (m < 0) return fail(RQ_EINVAL, "negative m");
    if (rank < 16 || rank > 64 || rank % 16)
        return fail(RQ_EINVAL, "rq_qmm_lora: rank must be 16, 32, 48 or 64 (got %lld)", (long long)rank);
    const int64_t n_out = transpose ? rows : cols;
    if (m == 0 || n_out == 0) return ok();
    const int64_t n_in = transpose ? cols : rows;
    if (n_in == 0) return fail(RQ_EINVAL, "rq_qmm_lora: empty contraction is not supported");
    if (!x || !w_q || !scales || !biases || !y || !z || !lora)
        return fail(RQ_EINVAL, "rq_qmm_lora: NULL pointer");
    if (!aligned16(x) || !aligned16(w_q) || !aligned16(z) || !aligned16(lora))
        return fail(RQ_EALIGN, "rq_qmm_lora: x, w_q, z and lora must be 16-byte aligned");
    const rq::LoraArgs lo{z, lora, (int)rank, scale};
    const hipError_t e = rq::launch_qmm(transpose, x, x_dt, w_q, scales, biases, sb_dt, m, rows,
                                        cols, group_size, bits, y, y_dt, (hipStream_t)stream, &lo);
    if (e == hipErrorNotSupported)
        return fail(RQ_EUNSUPPORTED,
                    "rq_qmm_lora: the fused low-rank term needs the 64-wide-stage GEMMs (bf16 or fp32 x, "
                    "m >= 256, 16-bit 16-byte aligned scales; transpose=1: cols a multiple of 8 "
                    "groups; transpose=0: rows %% 64 == 0, cols %% 128 == 0); use rq_qmm and add "
                    "the term separately");
    return launch_status(e, "rq_qmm_lora");
}

// The fused QLoRA products compute the down-projection once per output
// column tile: 12.5 % more MFMA work in every 128-column tile, on the waves
// that bound the GEMM.  Its rq_lora_down pass instead reads the activations
// once, so for outputs much wider than the contraction two launches cost
// less.  MI355X, M = 4096, inside the config-4 layer step (activations not
// cache-resident): dX of [2048, 8192] 180 us fused against 172 (a 7 us
// pass); the forward of [8192, 2048] 167 against 159 + 7 (its pass reads
// 16 MB at K = 2048, latency-bound).  Long contractions keep the fused
// kernels: a 64 MB pass costs 15-23 us there (dX of [8192, 2048] fused
// 150-155 against 139 + 23), and the [2048, 2048] products +5 us fused
// against +7.  bf16 or fp32 activations (the pass rounds fp32 ones to bf16
// as the GEMM does, so either gives the bits of bf16(x)), rank 16, 4 or 8
// bits, m >= 256: where the fused kernels apply.
static bool qlora_two_launch(int x_dt, int bits, int64_t rank, int64_t m, int64_t n_in,
                             int64_t n_out) {
    return (x_dt == RQ_BF16 || x_dt == RQ_F32) && (bits == 4 || bits == 8) && rank == 16 &&
           m >= 256 && n_in % 32 == 0 && n_out >= 4096 && n_out >= 2 * n_in;
}

int rq_qlora(const void* x, rq_dtype x_dt, const uint32_t* w_q, const void* scales,
             const void* biases, rq_dtype sb_dt, int64_t m, int64_t rows, int64_t cols,
             int group_size, int bits, int transpose, const void* a, const void* lora,
             int64_t rank, float scale, void* z_out, void* y, rq_dtype y_dt, void* stream) {
    if (int rc = check_common(rows, cols, group_size, bits)) return rc;
    if (!valid_dt(x_dt) || !valid_dt(sb_dt) || !valid_dt(y_dt)) return fail(RQ_EINVAL, "unsupported dtype");
    if (m < 0) return fail(RQ_EINVAL, "negative m");
    if (rank < 16 || rank > 64 || rank % 16)
        return fail(RQ_EINVAL, "rq_qlora: rank must be 16, 32, 48 or 64 (got %lld)", (long long)rank);
    const int64_t n_out = transpose ? rows : cols, n_in = transpose ? cols : rows;
    if (m == 0 || n_out == 0) return ok();
    if (n_in == 0) return fail(RQ_EINVAL, "rq_qlora: empty contraction is not supported");
    if (!x || !w_q || !scales || !biases || !y || !a || !lora)
        return fail(RQ_EINVAL, "rq_qlora: NULL pointer");
    if (!aligned16(x) || !aligned16(w_q) || !aligned16(a) || !aligned16(lora) || !aligned16(z_out))
        return fail(RQ_EALIGN, "rq_qlora: x, w_q, a, lora and z_out must be 16-byte aligned");
    hipError_t e;
    if (z_out && qlora_two_launch(x_dt, bits, rank, m, n_in, n_out)) {
        e = rq::launch_lora_down(x, m, n_in, a, (int)rank, z_out, (hipStream_t)stream,
                                 /*a_t=*/false, x_dt == RQ_F32);
        rq::LoraArgs lo{z_out, lora, (int)rank, scale};
        if (e == hipSuccess)
            e = rq::launch_qmm(transpose, x, x_dt, w_q, scales, biases, sb_dt, m, rows, cols,
                               group_size, bits, y, y_dt, (hipStream_t)stream, &lo);
    } else {
        rq::LoraArgs lo{nullptr, lora, (int)rank, scale};
        lo.a = a;
        lo.z_out = z_out;
        lo.a_ld = n_in;
        e = rq::launch_qmm(transpose, x, x_dt, w_q, scales, biases, sb_dt, m, rows, cols,
                           group_size, bits, y, y_dt, (hipStream_t)stream, &lo);
    }
    if (e == hipErrorNotSupported)
        return fail(RQ_EUNSUPPORTED,
                    "rq_qlora: the in-kernel down-projection covers rank 16 with 4- or 8-bit codes "
                    "on the 64-wide-stage GEMMs (bf16 or fp32 x, m >= 256, 16-bit 16-byte aligned scales; "
                    "transpose=1: cols a multiple of 8 groups; transpose=0: rows %% 64 == 0, "
                    "cols %% 128 == 0); use rq_lora_down and rq_qmm_lora");
    return launch_status(e, "rq_qlora");
}

int rq_qlora_dx(const void* dy, rq_dtype dy_dt, const uint32_t* w_q, const void* scales,
                const void* biases, rq_dtype sb_dt, int64_t m, int64_t rows, int64_t cols,
                int group_size, int bits, const void* lora_a, const void* lora_b, int64_t rank,
                float scale, void* u_out, void* dx, rq_dtype dx_dt, void* stream) {
    if (int rc = check_common(rows, cols, group_size, bits)) return rc;
    if (!valid_dt(dy_dt) || !valid_dt(sb_dt) || !valid_dt(dx_dt)) return fail(RQ_EINVAL, "unsupported dtype");
    if (m < 0) return fail(RQ_EINVAL, "negative m");
    if (rank < 16 || rank > 64 || rank % 16)
        return fail(RQ_EINVAL, "rq_qlora_dx: rank must be 16, 32, 48 or 64 (got %lld)", (long long)rank);
    if (m == 0 || cols == 0) return ok();
    if (rows == 0) return fail(RQ_EINVAL, "rq_qlora_dx: empty contraction is not supported");
    if (!dy || !w_q || !scales || !biases || !dx || !lora_a || !lora_b)
        return fail(RQ_EINVAL, "rq_qlora_dx: NULL pointer");
    // lora_b is read in 16-byte pieces (a stage's rows of B), lora_a in 2-byte ones
    if (!aligned16(dy) || !aligned16(w_q) || !aligned16(u_out) || !aligned16(lora_b))
        return fail(RQ_EALIGN, "rq_qlora_dx: dy, w_q, lora_b and u_out must be 16-byte aligned");
    if ((uintptr_t)lora_a & 1)
        return fail(RQ_EALIGN, "rq_qlora_dx: lora_a must be 2-byte aligned");
    // u = dY . B from B [rows, rank] as stored; the term scale * u . A from A
    // [rank, cols] as stored
    hipError_t e;
    if (u_out && qlora_two_launch(dy_dt, bits, rank, m, rows, cols)) {
        e = rq::launch_lora_down(dy, m, rows, lora_b, (int)rank, u_out, (hipStream_t)stream,
                                 /*a_t=*/true, dy_dt == RQ_F32);
        rq::LoraArgs lo{u_out, lora_a, (int)rank, scale};
        lo.stored = true;
        lo.l_ld = cols;
        if (e == hipSuccess)
            e = rq::launch_qmm(0, dy, dy_dt, w_q, scales, biases, sb_dt, m, rows, cols, group_size,
                               bits, dx, dx_dt, (hipStream_t)stream, &lo);
    } else {
        rq::LoraArgs lo{nullptr, lora_a, (int)rank, scale};
        lo.a = lora_b;
        lo.z_out = u_out;
        lo.a_ld = rows;
        lo.stored = true;
        lo.l_ld = cols;
        e = rq::launch_qmm(0, dy, dy_dt, w_q, scales, biases, sb_dt, m, rows, cols, group_size,
                           bits, dx, dx_dt, (hipStream_t)stream, &lo);
    }
    if (e == hipErrorNotSupported)
        return fail(RQ_EUNSUPPORTED,
                    "rq_qlora_dx: the in-kernel down-projection covers rank 16 with 4- or 8-bit "
                    "codes on the 64-wide-stage transposed GEMM (bf16 or fp32 dy, m >= 256, "
                    "16-bit 16-byte aligned scales, rows %% 64 == 0, cols %% 128 == 0); use "
                    "rq_lora_down and rq_qmm_lora");
    return launch_status(e, "rq_qlora_dx");
}

static int check_grouped(const char* what, const rq_problem* problems, int n, rq_dtype x_dt,
                         rq_dtype sb_dt, rq_dtype y_dt, int64_t m, int group_size, int bits) {
    if (n < 0 || (n > 0 && !problems)) return fail(RQ_EINVAL, "%s: bad problem list", what);
    if (!valid_dt(x_dt) || !valid_dt(sb_dt) || !valid_dt(y_dt)) return fail(RQ_EINVAL, "unsupported dtype");
    if (m < 1 || m > 16) return fail(RQ_EINVAL, "%s: m must be in [1, 16] (got %lld)", what, (long long)m);
    for (int i = 0; i < n; ++i) {
        const rq_problem& p = problems[i];
        if (int rc = check_common(p.rows, p.cols, group_size, bits)) return rc;
        if (p.cols == 0 && p.rows > 0)
            return fail(RQ_EINVAL, "%s: problem %d has an empty contraction", what, i);
        if (p.rows > 0 && (!p.x || !p.w_q || !p.scales || !p.biases || !p.y))
            return fail(RQ_EINVAL, "%s: NULL pointer in problem %d", what, i);
        if (!aligned16(p.x) || !aligned16(p.w_q))
            return fail(RQ_EALIGN, "%s: problem %d: x and w_q must be 16-byte aligned", what, i);
    }
    return RQ_OK;
}

int rq_qmm_grouped(const rq_problem* problems, int n, rq_dtype x_dt, rq_dtype sb_dt,
                   rq_dtype y_dt, int64_t m, int group_size, int bits, void* stream) {
    if (int rc = check_grouped("rq_qmm_grouped", problems, n, x_dt, sb_dt, y_dt, m, group_size, bits))
        return rc;
    if (n == 0) return ok();
    return launch_status(rq::launch_qmv(problems, n, x_dt, sb_dt, y_dt, m, group_size, bits,
                                        (hipStream_t)stream),
                         "rq_qmm_grouped");
}

// ---------------------------------------------------------------- plans
// Table layout in device memory: rq_problem descs[n] (sorted by cols,
// descending; 16-byte padded), then uint32 blocks[nblocks] with
// problem << 16 | 64-row block of that problem, longest blocks first.
static const int64_t kPlanMagic = 0x5251504c414e31ll;  // "RQPLAN1"

static int64_t plan_blocks(const rq_problem* problems, int n) {
    int64_t b = 0;
    for (int i = 0; i < n; ++i)
        b += (problems[i].rows + rq::kQmvRowsPerBlock - 1) / rq::kQmvRowsPerBlock;
    return b;
}

static int64_t plan_desc_bytes(int n) { return ((int64_t)n * (int64_t)sizeof(rq_problem) + 15) & ~15ll; }

int64_t rq_grouped_plan_table_bytes(const rq_problem* problems, int n) {
    if (n < 0 || (n > 0 && !problems)) return fail(RQ_EINVAL, "rq_grouped_plan_table_bytes: bad problem list");
    return plan_desc_bytes(n) + 4 * plan_blocks(problems, n);
}

int rq_grouped_plan_init(const rq_problem* problems, int n, rq_dtype x_dt, rq_dtype sb_dt,
                         rq_dtype y_dt, int64_t m, int group_size, int bits, void* table,
                         int64_t table_bytes, rq_grouped_plan* plan, void* stream) {
    if (!plan) return fail(RQ_EINVAL, "rq_grouped_plan_init: NULL plan");
    std::memset(plan, 0, sizeof(*plan));
    if (int rc = check_grouped("rq_grouped_plan_init", problems, n, x_dt, sb_dt, y_dt, m,
                               group_size, bits))
        return rc;
    const int64_t mk = rq::qmv_rows(x_dt, m);  // MFMA activation rows
    std::vector<int> order;
    for (int i = 0; i < n; ++i) {
        if (problems[i].rows == 0) continue;
        if (!rq::qmv_stream_covers(problems[i], sb_dt, mk, group_size, bits))
            return fail(RQ_EUNSUPPORTED,
                        "rq_grouped_plan_init: problem %d is outside the planned GEMV (needs "
                        "16-bit scales, cols %% 512 == 0, 16-byte aligned scales/biases, and "
                        "either m <= 4 with m*cols*2 bytes of activations within the LDS budget "
                        "or 4 < m <= 16 with 4- or 8-bit codes); use rq_qmm_grouped",
                        i);
        if ((problems[i].rows + rq::kQmvRowsPerBlock - 1) / rq::kQmvRowsPerBlock > 65536)
            return fail(RQ_EUNSUPPORTED, "rq_grouped_plan_init: problem %d has too many rows", i);
        order.push_back(i);
    }
    if (order.size() > 65535) return fail(RQ_EUNSUPPORTED, "rq_grouped_plan_init: too many problems");
    // longest contraction first: the last blocks to start are the shortest
    std::stable_sort(order.begin(), order.end(),
                     [&](int a, int b) { return problems[a].cols > problems[b].cols; });
    const int nn = (int)order.size();
    std::vector<rq_problem> descs(nn);
    size_t lds = 0;
    for (int i = 0; i < nn; ++i) {
        descs[i] = problems[order[i]];
        lds = std::max(lds, rq::qmv_stream_lds(mk, descs[i].cols, group_size, bits));
    }
    const int64_t nblocks = plan_blocks(descs.data(), nn);
    const int64_t dbytes = plan_desc_bytes(nn);
    const int64_t need = dbytes + 4 * nblocks;
    if (nn > 0) {
        if (!table) return fail(RQ_EINVAL, "rq_grouped_plan_init: NULL table");
        if (!aligned16(table)) return fail(RQ_EALIGN, "rq_grouped_plan_init: table must be 16-byte aligned");
        if (table_bytes < need)
            return fail(RQ_EINVAL, "rq_grouped_plan_init: table has %lld bytes, needs %lld",
                        (long long)table_bytes, (long long)need);
        std::vector<uint8_t> host((size_t)need, 0);
        std::memcpy(host.data(), descs.data(), (size_t)nn * sizeof(rq_problem));
        uint32_t* blk = (uint32_t*)(host.data() + dbytes);
        int64_t b = 0;
        for (int i = 0; i < nn; ++i) {
            const int64_t nb = (descs[i].rows + rq::kQmvRowsPerBlock - 1) / rq::kQmvRowsPerBlock;
            for (int64_t j = 0; j < nb; ++j) blk[b++] = ((uint32_t)i << 16) | (uint32_t)j;
        }
        hipStream_t s = (hipStream_t)stream;
        hipError_t e = hipMemcpyAsync(table, host.data(), (size_t)need, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);  // the host copy dies with this call
        if (e != hipSuccess)
            return fail(RQ_ELAUNCH, "rq_grouped_plan_init: table upload failed: %s", hipGetErrorString(e));
    }
    plan->opaque[0] = (int64_t)(uintptr_t)table;
    plan->opaque[1] = nblocks;
    plan->opaque[2] = m;
    plan->opaque[3] = group_size;
    plan->opaque[4] = bits;
    plan->opaque[5] = (int64_t)x_dt | ((int64_t)sb_dt << 8) | ((int64_t)y_dt << 16) | ((int64_t)nn << 24);
    plan->opaque[6] = (int64_t)lds;
    plan->opaque[7] = kPlanMagic;
    return ok();
}

int rq_grouped_plan_run(const rq_grouped_plan* plan, void* stream) {
    if (!plan || plan->opaque[7] != kPlanMagic)
        return fail(RQ_EINVAL, "rq_grouped_plan_run: not an initialised plan");
    const int64_t nblocks = plan->opaque[1];
    if (nblocks == 0) return ok();
    const int nn = (int)(plan->opaque[5] >> 24);
    rq::QmvTable t;
    t.descs = (const rq_problem*)(uintptr_t)plan->opaque[0];
    t.blocks = (const uint32_t*)((const uint8_t*)t.descs + plan_desc_bytes(nn));
    t.x_dt = (int)(plan->opaque[5] & 0xff);
    t.xsplit = rq::qmv_xsplit(t.x_dt, plan->opaque[2]) ? 1 : 0;
    t.m = (int)rq::qmv_rows(t.x_dt, plan->opaque[2]);
    t.y_dt = (int)((plan->opaque[5] >> 16) & 0xff);
    const int sb_dt = (int)((plan->opaque[5] >> 8) & 0xff);
    return launch_status(rq::launch_qmv_table(t, (int)nblocks, sb_dt, (int)plan->opaque[3],
                                              (int)plan->opaque[4], (size_t)plan->opaque[6],
                                              (hipStream_t)stream),
                         "rq_grouped_plan_run");
}

}  // extern "C"
