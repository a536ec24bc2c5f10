// rq_qmm.hip -- prefill / backward GEMMs on group-affine packed weights (gfx950).
//
//   qmm_t : y[m, r] = sum_k x[m, k] * ŵ[r, k]     (transpose=True,  forward)
//   qmm_n : y[m, k] = sum_r x[m, r] * ŵ[r, k]     (transpose=False, dX = dY·W)
//
// mx.quantized_matmul at prefill sizes (rwkv_metal/lora/rwkvq_native.py:120-122,
// QuantizedLinear inside LoRALinear, rwkv_metal/lora/lora.py:58-59) and its VJP
// w.r.t. x, which MLX autograd emits for the QLoRA backward
// (rwkv_metal/lora/finetune.py:141).
//
// Design: block tile BM x 128 outputs, 64 contraction elements per stage,
// 4 waves in a 2x2 arrangement, v_mfma_f32_16x16x32_bf16 with fp32
// accumulators.  Packed weights are dequantized ONCE per block per stage in
// registers (ŵ = bf16(fma(scale, code, bias))) and written to LDS as bf16;
// the activation tile is converted to bf16 on its way to LDS.  LDS is double
// buffered and the next stage's global loads are issued before the current
// stage's MFMAs.
//
//  * qmm_t: the packed axis K is the contraction axis, so a thread's 32-code
//    run lands as one 64-byte row segment of the B tile (row-major [n][k]).
//  * qmm_n: the contraction runs over the weight rows, so the B tile is
//    stored transposed ([k][r]); a thread dequantizes the same run of two
//    adjacent rows and writes (row, row+1) pairs as one dword per k.
#include "rq_common.h"
#include "rq_launch.h"

#ifndef RQ_BITS
#error "compile rq_qmm.hip once per bit width with -DRQ_BITS=<bits>"
#endif

namespace {

constexpr int kBlock = 256;
constexpr int BK = 64;        // contraction elements per stage
constexpr int LDS_LD = BK + 8;  // LDS row stride in bf16 elements (144 B)
constexpr int BN = 128;       // output columns per block

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

RQ_DEV bf16x8_t lds_frag(const uint16_t* p) {
    return __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)p);
}

// One run of 32 codes -> 16 dwords of bf16 pairs, ŵ = bf16(scale*code + bias).
template <int BITS>
RQ_DEV void dequant_run_bf16(const uint32_t* words, float s, float b, uint32_t* out) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float lo = fmaf(s, (float)run_code<BITS>(words, 2 * i), b);
        const float hi = fmaf(s, (float)run_code<BITS>(words, 2 * i + 1), b);
        out[i] = pack_bf16x2(lo, hi);
    }
}

// Load 32 activations x[row][col0 .. col0+31] (row length ld elements) as 16
// bf16-pair dwords; elements at col >= ncols are zero.  `vec` selects 128-bit
// loads (the caller guarantees alignment and that the run is in bounds).
template <int XDT>
RQ_DEV void load_act_run(const void* x, int64_t row, int64_t ld, int64_t col0, int64_t ncols,
                         bool vec, uint32_t* d) {
    if (vec) {
        const int64_t off = row * ld + col0;
        if constexpr (XDT == RQ_BF16) {
            const uint4* p = (const uint4*)((const uint16_t*)x + off);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint4 v = p[i];
                d[4 * i] = v.x; d[4 * i + 1] = v.y; d[4 * i + 2] = v.z; d[4 * i + 3] = v.w;
            }
        } else {
            float f[32];
            load32_f32<XDT>(x, off, f);
#pragma unroll
            for (int i = 0; i < 16; ++i) d[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
        }
    } else {
        typedef typename dt_traits<XDT>::storage S;
        const S* px = (const S*)x + row * ld;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int64_t c = col0 + 2 * i;
            const float lo = c < ncols ? dt_traits<XDT>::to_f32(px[c]) : 0.f;
            const float hi = c + 1 < ncols ? dt_traits<XDT>::to_f32(px[c + 1]) : 0.f;
            d[i] = pack_bf16x2(lo, hi);
        }
    }
}

RQ_DEV void store_16dw(uint16_t* lds, const uint32_t* d) {
    u32x4_t* p = (u32x4_t*)lds;
#pragma unroll
    for (int q = 0; q < 4; ++q) p[q] = u32x4_t{d[4 * q], d[4 * q + 1], d[4 * q + 2], d[4 * q + 3]};
}

// ----------------------------------------------------------------- qmm_t

template <int BITS, int XDT, int BM>
__global__ __launch_bounds__(kBlock) void qmm_t_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, int sb_dt, int64_t M, int64_t R, int64_t K, int gs_shift,
    void* __restrict__ y, int y_dt) {
    constexpr int TM = BM / 32;  // 16-row MFMA tiles per wave along m (wave covers BM/2)
    constexpr int TN = 4;        // wave covers 64 output columns
    constexpr int AR = BM / 128; // activation rows loaded per thread per stage
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDS_LD];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDS_LD];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lg = lane >> 4, lr = lane & 15;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int64_t runs_per_row = K >> 5, wpr = runs_per_row * BITS, G = K >> gs_shift;
    const int nst = (int)((runs_per_row + 1) >> 1);
    const int half = tid & 1;           // which run of the stage this thread loads
    const int64_t brow = n0 + (tid >> 1);

    uint32_t cw[BITS];
    float sc = 0.f, bi = 0.f;
    uint32_t xa[AR][16];

    auto gload = [&](int st) {
        const int64_t run = 2 * (int64_t)st + half;
        const bool run_ok = run < runs_per_row;
        if (run_ok && brow < R) {
            load_run<BITS>(wq + brow * wpr + run * BITS, cw);
            const int64_t gi = brow * G + (run >> (gs_shift - 5));
            sc = load_dt(scales, sb_dt, gi);
            bi = load_dt(biases, sb_dt, gi);
        } else {
#pragma unroll
            for (int w = 0; w < BITS; ++w) cw[w] = 0u;
            sc = 0.f;
            bi = 0.f;
        }
#pragma unroll
        for (int i = 0; i < AR; ++i) {
            const int64_t arow = m0 + (tid >> 1) + 128 * i;
            if (run_ok && arow < M) {
                load_act_run<XDT>(x, arow, K, run * 32, K, true, xa[i]);
            } else {
#pragma unroll
                for (int q = 0; q < 16; ++q) xa[i][q] = 0u;
            }
        }
    };
    auto swrite = [&](int buf) {
        uint32_t d[16];
        dequant_run_bf16<BITS>(cw, sc, bi, d);
        store_16dw(&Bs[buf][(tid >> 1) * LDS_LD + half * 32], d);
#pragma unroll
        for (int i = 0; i < AR; ++i)
            store_16dw(&As[buf][((tid >> 1) + 128 * i) * LDS_LD + half * 32], xa[i]);
    };

    f32x4_t acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    gload(0);
    swrite(0);
    __syncthreads();
    for (int st = 0; st < nst; ++st) {
        const int buf = st & 1;
        if (st + 1 < nst) gload(st + 1);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            bf16x8_t af[TM], bf[TN];
#pragma unroll
            for (int a = 0; a < TM; ++a)
                af[a] = lds_frag(&As[buf][(wm * (BM / 2) + a * 16 + lr) * LDS_LD + ks * 32 + lg * 8]);
#pragma unroll
            for (int b = 0; b < TN; ++b)
                bf[b] = lds_frag(&Bs[buf][(wn * 64 + b * 16 + lr) * LDS_LD + ks * 32 + lg * 8]);
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[a], bf[b], acc[a][b],
                                                                        0, 0, 0);
        }
        if (st + 1 < nst) swrite(buf ^ 1);
        __syncthreads();
    }

    // D[4*lg + i][lr] of each 16x16 tile: rows are m, columns are n.
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int64_t n = n0 + wn * 64 + b * 16 + lr;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t m = m0 + wm * (BM / 2) + a * 16 + 4 * lg + i;
                if (m < M && n < R) store_dt(y, y_dt, m * R + n, acc[a][b][i]);
            }
        }
}

// ----------------------------------------------------------------- qmm_n

template <int BITS, int XDT, int BM>
__global__ __launch_bounds__(kBlock) void qmm_n_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, int sb_dt, int64_t M, int64_t R, int64_t K, int gs_shift,
    void* __restrict__ y, int y_dt, int x_vec) {
    constexpr int TM = BM / 32;
    constexpr int TN = 4;
    constexpr int AU = BM / 64;  // activation row-runs per A-loader thread (128 threads)
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDS_LD];  // [m][r]
    __shared__ __attribute__((aligned(16))) uint16_t Bt[2][BN * LDS_LD];  // [k][r]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lg = lane >> 4, lr = lane & 15;
    const int64_t m0 = (int64_t)blockIdx.y * BM, k0 = (int64_t)blockIdx.x * BN;
    const int64_t runs_per_row = K >> 5, wpr = runs_per_row * BITS, G = K >> gs_shift;
    const int nst = (int)((R + BK - 1) / BK);
    const bool is_b = tid < 128;  // waves 0-1 dequantize weights, waves 2-3 load x

    // B unit: rows (2*pr, 2*pr+1) of the stage, run q of the block's 4 runs.
    const int pr = tid & 31, q = (tid >> 5) & 3;
    const int64_t brun = (k0 >> 5) + q;
    // A unit(s): activation row ua/2 (+64 per extra unit), half ua&1 of the 64 r.
    const int ua = tid - 128;

    uint32_t cw[2][BITS];
    float sc[2] = {0.f, 0.f}, bi[2] = {0.f, 0.f};
    uint32_t xa[AU][16];

    auto gload = [&](int st) {
        const int64_t r0 = (int64_t)st * BK;
        if (is_b) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int64_t r = r0 + 2 * pr + h;
                if (r < R && brun < runs_per_row) {
                    load_run<BITS>(wq + r * wpr + brun * BITS, cw[h]);
                    const int64_t gi = r * G + (brun >> (gs_shift - 5));
                    sc[h] = load_dt(scales, sb_dt, gi);
                    bi[h] = load_dt(biases, sb_dt, gi);
                } else {
#pragma unroll
                    for (int w = 0; w < BITS; ++w) cw[h][w] = 0u;
                    sc[h] = 0.f;
                    bi[h] = 0.f;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < AU; ++i) {
                const int64_t arow = m0 + (ua >> 1) + 64 * i;
                const int64_t c0 = r0 + (ua & 1) * 32;
                if (arow < M && c0 < R) {
                    const bool vec = x_vec && (c0 + 32 <= R);
                    load_act_run<XDT>(x, arow, R, c0, R, vec, xa[i]);
                } else {
#pragma unroll
                    for (int t = 0; t < 16; ++t) xa[i][t] = 0u;
                }
            }
        }
    };
    auto swrite = [&](int buf) {
        if (is_b) {
            // Dequantize both rows and write (row, row+1) pairs down column k.
#pragma unroll
            for (int j = 0; j < 32; ++j) {
                const float v0 = fmaf(sc[0], (float)run_code<BITS>(cw[0], j), bi[0]);
                const float v1 = fmaf(sc[1], (float)run_code<BITS>(cw[1], j), bi[1]);
                *(uint32_t*)&Bt[buf][(q * 32 + j) * LDS_LD + 2 * pr] = pack_bf16x2(v0, v1);
            }
        } else {
#pragma unroll
            for (int i = 0; i < AU; ++i)
                store_16dw(&As[buf][((ua >> 1) + 64 * i) * LDS_LD + (ua & 1) * 32], xa[i]);
        }
    };

    f32x4_t acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    gload(0);
    swrite(0);
    __syncthreads();
    for (int st = 0; st < nst; ++st) {
        const int buf = st & 1;
        if (st + 1 < nst) gload(st + 1);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            bf16x8_t af[TM], bf[TN];
#pragma unroll
            for (int a = 0; a < TM; ++a)
                af[a] = lds_frag(&As[buf][(wm * (BM / 2) + a * 16 + lr) * LDS_LD + ks * 32 + lg * 8]);
#pragma unroll
            for (int b = 0; b < TN; ++b)
                bf[b] = lds_frag(&Bt[buf][(wn * 64 + b * 16 + lr) * LDS_LD + ks * 32 + lg * 8]);
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[a], bf[b], acc[a][b],
                                                                        0, 0, 0);
        }
        if (st + 1 < nst) swrite(buf ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int64_t n = k0 + wn * 64 + b * 16 + lr;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t m = m0 + wm * (BM / 2) + a * 16 + 4 * lg + i;
                if (m < M && n < K) store_dt(y, y_dt, m * K + n, acc[a][b][i]);
            }
        }
}

}  // namespace

namespace rq {

#define RQ_CAT2(a, b) a##b
#define RQ_CAT(a, b) RQ_CAT2(a, b)

hipError_t RQ_CAT(launch_qmm_t_b, RQ_BITS)(const void* x, int x_dt, const uint32_t* wq,
                                      const void* scales, const void* biases, int sb_dt,
                                      int64_t m, int64_t rows, int64_t cols, int gs, void* y,
                                      int y_dt, hipStream_t stream) {
    constexpr int BM = 128;
    const dim3 grid((unsigned)((rows + BN - 1) / BN), (unsigned)((m + BM - 1) / BM));
    const int gs_shift = __builtin_ctz(gs);
    RQ_DISPATCH_DT(x_dt, XD,
        hipLaunchKernelGGL((qmm_t_kernel<RQ_BITS, XD, BM>), grid, dim3(kBlock), 0, stream, x, wq,
                           scales, biases, sb_dt, m, rows, cols, gs_shift, y, y_dt));
    return hipGetLastError();
}

hipError_t RQ_CAT(launch_qmm_n_b, RQ_BITS)(const void* x, int x_dt, const uint32_t* wq,
                                      const void* scales, const void* biases, int sb_dt,
                                      int64_t m, int64_t rows, int64_t cols, int gs, void* y,
                                      int y_dt, hipStream_t stream) {
    constexpr int BM = 128;
    const dim3 grid((unsigned)((cols + BN - 1) / BN), (unsigned)((m + BM - 1) / BM));
    const int gs_shift = __builtin_ctz(gs);
    // 128-bit activation loads need every 32-element run of a row 16-byte aligned.
    const int esz = x_dt == RQ_F32 ? 4 : 2;
    const int x_vec = ((rows * esz) % 16 == 0) && (((uintptr_t)x & 15) == 0);
    RQ_DISPATCH_DT(x_dt, XD,
        hipLaunchKernelGGL((qmm_n_kernel<RQ_BITS, XD, BM>), grid, dim3(kBlock), 0, stream, x, wq,
                           scales, biases, sb_dt, m, rows, cols, gs_shift, y, y_dt, x_vec));
    return hipGetLastError();
}

}  // namespace rq
