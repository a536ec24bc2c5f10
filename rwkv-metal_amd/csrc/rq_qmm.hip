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
#include <type_traits>

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


// ------------------------------------------------------------- qmm_t_big
//
// Large-M forward GEMM.  Block tile 256 (activation rows) x BN (weight rows),
// 64 contraction elements per stage, four waves in a 2x2 arrangement with a
// 128 x BN/2 wave tile of 16x16x32 bf16 MFMAs (fp32 accumulators).  BN is
// chosen per shape so that an M=4096 problem fills the 256 CUs in whole
// rounds (BN=160 for N in {2560, 10240}, BN=128 otherwise).  Each stage: the block's packed weight tile is dequantized once
// (fp32 fma of scale, code and bias, rounded to bf16) and written to LDS
// next to the bf16 activation tile; LDS is double buffered and the next
// stage's global loads are issued before the current stage's MFMAs.
// Blocks are assigned to tiles so that each XCD works on a contiguous run of
// tiles (shared activation rows and weight rows stay in that XCD's L2).

// Eight 4-bit codes of one word -> 4 dwords of bf16 pairs (codes 0,1 .. 6,7),
// ŵ = bf16(s*code + b).  gfx950's v_cvt_scalef32_pk_f32_fp8 turns two bytes
// into two fp32 values in one instruction: an e4m3 byte 0x0q is exactly
// q / 512 (its subnormals and first binade are evenly spaced, 2^-9 apart),
// and the conversion applies only the exponent of its scale (measured on
// the box), so a scale of 512 gives q exactly.  Per 8 codes: 3 mask ops, 4
// converts, 8 fmas, 4 packs (byte converts took 8 converts).
RQ_DEV void dequant_word4(uint32_t word, float s, float b, uint32_t* out) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    const uint32_t lo = word & 0x0F0F0F0Fu;         // codes 0,2,4,6
    const uint32_t hi = (word >> 4) & 0x0F0F0F0Fu;  // codes 1,3,5,7
    const f32x2_t l0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(lo, 512.f, false);
    const f32x2_t l1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(lo, 512.f, true);
    const f32x2_t h0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 512.f, false);
    const f32x2_t h1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hi, 512.f, true);
    out[0] = pack_bf16x2(fmaf(s, l0[0], b), fmaf(s, h0[0], b));
    out[1] = pack_bf16x2(fmaf(s, l0[1], b), fmaf(s, h0[1], b));
    out[2] = pack_bf16x2(fmaf(s, l1[0], b), fmaf(s, h1[0], b));
    out[3] = pack_bf16x2(fmaf(s, l1[1], b), fmaf(s, h1[1], b));
}

// One run of 32 codes -> 16 dwords of bf16 pairs, ŵ = bf16(scale*code + bias):
// 4-bit codes by dequant_word4, 8-bit ones by byte converts
// (v_cvt_f32_ubyte0..3; the bytes are hidden from the optimiser by an empty
// asm, otherwise it folds each byte select into a bit-field extract, a second
// VALU op per code in front of a v_cvt_f32_ubyte0).
template <int BITS>
RQ_DEV void dequant_run_fast(const uint32_t* words, float s, float b, uint32_t* out) {
    if constexpr (BITS == 4) {
#pragma unroll
        for (int w = 0; w < 4; ++w) dequant_word4(words[w], s, b, out + 4 * w);
    } else if constexpr (BITS == 8) {
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            uint32_t v = words[w];
            asm("" : "+v"(v));
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const float c0 = (float)(uint8_t)(v >> (16 * i));
                const float c1 = (float)(uint8_t)(v >> (16 * i + 8));
                out[2 * w + i] = pack_bf16x2(fmaf(s, c0, b), fmaf(s, c1, b));
            }
        }
    } else {
        dequant_run_bf16<BITS>(words, s, b, out);
    }
}

template <int BITS, int XDT, int BN>
__global__ __launch_bounds__(kBlock, 1) void qmm_t_big(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, int sb_dt, int64_t M, int64_t R, int64_t K, int gs_shift,
    void* __restrict__ y, int y_dt, int tiles_m, int tiles_n) {
    constexpr int BM = 256;
    constexpr int WN = BN / 2;           // wave tile: 128 x WN
    constexpr int TM = 8, TN = WN / 16;  // 16x16 MFMA tiles per wave
    constexpr int NRUN = (2 * BN + kBlock - 1) / kBlock;  // weight runs per thread per stage
    constexpr int TILE_ELEMS = (BM + BN) * LDS_LD;
    __shared__ __attribute__((aligned(16))) uint16_t smem[2 * TILE_ELEMS];

    // XCD-aware tile order: consecutive block ids go to different XCDs, so
    // block b works on tile (b % 8) * per_xcd + b / 8.
    const int ntiles = tiles_m * tiles_n;
    const int per_xcd = (ntiles + 7) / 8;
    const int t = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
    if (t >= ntiles) return;
    const int64_t m0 = (int64_t)(t / tiles_n) * BM, n0 = (int64_t)(t % tiles_n) * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lg = lane >> 4, lr = lane & 15;
    const int64_t runs_per_row = K >> 5, wpr = runs_per_row * BITS, G = K >> gs_shift;
    const int nst = (int)((runs_per_row + 1) >> 1);

    // activation tile: 256 rows x 64 k = 2048 16-byte chunks of bf16, 8 per thread
    uint32_t xa[8][4];
    uint32_t cw[NRUN][BITS];
    float sc[NRUN], bi[NRUN];

    auto gload = [&](int st) {
        const int64_t k0 = (int64_t)st * BK;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int c = tid + kBlock * i;
            const int64_t row = m0 + (c >> 3);
            const int64_t col = k0 + (c & 7) * 8;
            if (row < M && col < K) {
                if constexpr (XDT == RQ_BF16) {
                    const uint4 v = *(const uint4*)((const uint16_t*)x + row * K + col);
                    xa[i][0] = v.x; xa[i][1] = v.y; xa[i][2] = v.z; xa[i][3] = v.w;
                } else {
                    typedef typename dt_traits<XDT>::storage S;
                    const S* px = (const S*)x + row * K + col;
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        xa[i][q] = pack_bf16x2(dt_traits<XDT>::to_f32(px[2 * q]),
                                               dt_traits<XDT>::to_f32(px[2 * q + 1]));
                }
            } else {
                xa[i][0] = xa[i][1] = xa[i][2] = xa[i][3] = 0u;
            }
        }
#pragma unroll
        for (int i = 0; i < NRUN; ++i) {
            const int r = tid + kBlock * i;
            const int64_t row = n0 + (r >> 1);
            const int64_t run = 2 * (int64_t)st + (r & 1);
            if (r < 2 * BN && row < R && run < runs_per_row) {
                load_run<BITS>(wq + row * wpr + run * BITS, cw[i]);
                const int64_t gi = row * G + (run >> (gs_shift - 5));
                sc[i] = load_dt(scales, sb_dt, gi);
                bi[i] = load_dt(biases, sb_dt, gi);
            } else {
#pragma unroll
                for (int w = 0; w < BITS; ++w) cw[i][w] = 0u;
                sc[i] = 0.f;
                bi[i] = 0.f;
            }
        }
    };
    auto swrite = [&](int buf) {
        uint16_t* As = smem + buf * TILE_ELEMS;
        uint16_t* Bs = As + BM * LDS_LD;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int c = tid + kBlock * i;
            *(u32x4_t*)&As[(c >> 3) * LDS_LD + (c & 7) * 8] =
                u32x4_t{xa[i][0], xa[i][1], xa[i][2], xa[i][3]};
        }
#pragma unroll
        for (int i = 0; i < NRUN; ++i) {
            const int r = tid + kBlock * i;
            if (r < 2 * BN) {
                uint32_t d[16];
                dequant_run_fast<BITS>(cw[i], sc[i], bi[i], d);
                store_16dw(&Bs[(r >> 1) * LDS_LD + (r & 1) * 32], d);
            }
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
        const uint16_t* As = smem + buf * TILE_ELEMS;
        const uint16_t* Bs = As + BM * LDS_LD;
        if (st + 1 < nst) gload(st + 1);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            bf16x8_t af[TM], bf[TN];
#pragma unroll
            for (int a = 0; a < TM; ++a)
                af[a] = lds_frag(&As[(wm * 128 + a * 16 + lr) * LDS_LD + ks * 32 + lg * 8]);
#pragma unroll
            for (int b = 0; b < TN; ++b)
                bf[b] = lds_frag(&Bs[(wn * WN + b * 16 + lr) * LDS_LD + ks * 32 + lg * 8]);
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
            const int64_t n = n0 + wn * WN + b * 16 + lr;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t m = m0 + wm * 128 + a * 16 + 4 * lg + i;
                if (m < M && n < R) store_dt(y, y_dt, m * R + n, acc[a][b][i]);
            }
        }
}


// ------------------------------------------------- direct-to-LDS helpers

typedef __attribute__((address_space(3))) void lds_void_t;

template <int N>
RQ_DEV void s_wait_vmcnt_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] (7 = no wait) | lgkmcnt[11:8] | vmcnt[5:4] << 14
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}

// -------------------------------------------------------------- qmm_t_ws
//
// Warp-specialised GEMM fed by direct-to-LDS loads (global_load_lds; bf16
// activations, M >= 256, the cases qmm_t_k64 does not take: fp32 scales,
// K not a multiple of 8 groups, unaligned scales).  32-element stages of
// 256 activation rows x 64 bytes (16-byte chunks XOR-swizzled) and the BN
// rows' codes and (scale, bias) arrive in an LDS ring, ring-depth-1 stages
// ahead, with no staging registers.  8 waves per block.  Waves 0-3 only run
// MFMAs (2x2, wave tile 128 x BN/2, fp32 accumulators); waves 4-7
// ("producers") issue every direct-to-LDS load of the ring and dequantize one
// stage ahead.  Each SIMD holds one wave of
// each kind, so the hardware interleaves the producers' VALU work with the
// consumers' matrix instructions.  One workgroup barrier per stage of 32
// contraction elements orders the rings:
//   producers: wait own DMAs of stage st+1 and own LDS writes; barrier;
//              DMA stage st+AHEAD; dequantize stage st+1 into bf16 slot.
//   consumers: wait own LDS reads; barrier; MFMAs on stage st.
constexpr int kWsBlock = 512;
#ifndef RQ_K64_DEPTH
#define RQ_K64_DEPTH 2  // qmm_t_k64: stages of loads in flight per producer thread
#endif
#ifndef RQ_K64_SB64
#define RQ_K64_SB64 2  // qmm_t_k64, 64 x 96 tiles: 64-wide stages per barrier
#endif
#ifndef RQ_K64_SB128
#define RQ_K64_SB128 1  // qmm_t_k64, 128 x 128 tiles: 64-wide stages per barrier
#endif
#ifndef RQ_K64_PPRIO
#define RQ_K64_PPRIO 2  // qmm_t_k64: wave priority of the producer waves (0-3; 2 measured +4-6%)
#endif
#ifndef RQ_K64_BM128_BELOW
#define RQ_K64_BM128_BELOW 200  // qmm_t_k64: 128-row tiles when 256-row ones number fewer
#endif
#ifndef RQ_K64_BM64_BELOW
#define RQ_K64_BM64_BELOW 128  // qmm_t_k64, 4 bits: 64 x 96 tiles when 128-row ones number fewer
#endif
#ifndef RQ_K64_CPRIO
#define RQ_K64_CPRIO 0  // qmm_t_k64: wave priority of the MFMA waves (0-3)
#endif
#ifndef RQ_K64_GROUP
#define RQ_K64_GROUP 2  // qmm_t_k64: row tiles per group of the tile order (1: row-major)
#endif
// tile index -> (row tile, column tile): groups of RQ_K64_GROUP row tiles
// walked column by column (a bijection; the last group may be shorter)
__device__ __forceinline__ void k64_tile(int t, int tiles_m, int tiles_n, int& mt, int& nt) {
    constexpr int G = RQ_K64_GROUP;
    if (G == 1) {
        mt = t / tiles_n;
        nt = t % tiles_n;
        return;
    }
    const int group = t / (G * tiles_n), first = group * G;
    const int gsz = tiles_m - first < G ? tiles_m - first : G;
    const int r = t - group * G * tiles_n;
    mt = first + r % gsz;
    nt = r / gsz;
}
#ifndef RQ_GEMM_K64
#define RQ_GEMM_K64 1  // 1: 64-wide stages with whole-line loads (qmm_t_k64) where they apply
#endif
#ifndef RQ_GEMM_N160
#define RQ_GEMM_N160 1  // 1: 160-column tiles for the transposed GEMM where they fill the GPU better
#endif
constexpr int kK64Cus = 256;  // CUs of one MI355X: one k64 block per CU
#ifndef RQ_WS_SLOTS
#define RQ_WS_SLOTS 6  // DMA ring slots of qmm_t_ws (4 or 6): RQ_WS_SLOTS-1 stages in flight
#endif

template <int BITS, int SDT, int BN, int NSLOT, bool SBP>
struct WsCfg {
    static constexpr int BM = 256;
    static constexpr int AHEAD = NSLOT - 1;
    static constexpr int NP = 256;                              // producer threads
    static constexpr int X_BYTES = BM * 64;                     // 16 KB activation stage
    static constexpr int NX = X_BYTES / (NP * 16);              // 4 x-DMAs per producer
    static constexpr int CODE_DW = BN * BITS;
    static constexpr int NC = (CODE_DW + NP - 1) / NP;          // code DMAs per producer
    static constexpr int C_BYTES = NC * NP * 4;
    static constexpr int SB = SDT == RQ_F32 ? 4 : 2;
    // SBP: the (scale, bias) values of 8 groups per row arrive with one
    // 16-byte DMA each per 8 groups, one period ahead, and are copied to the
    // buffer the dequantisation reads at the period start; otherwise one 2-
    // or 4-byte DMA each per stage.
    static constexpr int S_BYTES = SBP ? 16 : NP * 4;           // 4-byte lane stride
    static constexpr int PER_STAGE = NX + NC + (SBP ? 0 : 2);
    static constexpr int SBP_BYTES = SBP ? BN * 16 : 16;        // per row and buffer: 8 values
    static constexpr int BLD = 40;                              // bf16 ring row stride
    static constexpr int B_BYTES = BN * BLD * 2;
    static_assert(NSLOT % 2 == 0, "the bf16 ring index is derived from the slot index");
    static_assert(BN <= NP, "one producer thread dequantizes one weight row");
};

// LDS bytes of qmm_t_ws (the slot arrays, the bf16 ring and the scale buffers).
template <int BITS, int SDT, int BN, int NSLOT, bool SBP>
constexpr size_t ws_lds_bytes() {
    typedef WsCfg<BITS, SDT, BN, NSLOT, SBP> C;
    return (size_t)NSLOT * (C::X_BYTES + C::C_BYTES + 2 * C::S_BYTES) + (6 - NSLOT) * 4 * 16 +
           2 * (size_t)BN * C::BLD * 2 + 4 * (size_t)C::SBP_BYTES;
}
// The deepest ring that fits the 160 KB of LDS.
template <int BITS, int SDT, int BN, bool SBP>
constexpr int ws_slots() {
    return (RQ_WS_SLOTS >= 6 && ws_lds_bytes<BITS, SDT, BN, 6, SBP>() <= 160 * 1024) ? 6 : 4;
}

template <int BITS, int SDT, int BN, int NSLOT, bool SBP>
__global__ __launch_bounds__(kWsBlock, 1) void qmm_t_ws(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, int64_t M, int64_t R, int64_t K, int gs_shift,
    void* __restrict__ y, int y_dt, int tiles_m, int tiles_n) {
    typedef WsCfg<BITS, SDT, BN, NSLOT, SBP> C;
    static_assert(!SBP || SDT != RQ_F32, "parked scales are 16-bit");
    constexpr int BM = C::BM;
    constexpr int WN = BN / 2;
    constexpr int TM = 8, TN = WN / 16;
    // One __shared__ object per ring slot (up to 6; slots >= NSLOT are 16-byte
    // stubs), so that the compiler can tell a DMA's target from the slots
    // being read and never makes a read wait for a DMA in flight.
#define RQ_RING(name, bytes)                                                              \
    __shared__ __attribute__((aligned(16))) uint8_t name##0[bytes];                       \
    __shared__ __attribute__((aligned(16))) uint8_t name##1[bytes];                       \
    __shared__ __attribute__((aligned(16))) uint8_t name##2[bytes];                       \
    __shared__ __attribute__((aligned(16))) uint8_t name##3[bytes];                       \
    __shared__ __attribute__((aligned(16))) uint8_t name##4[NSLOT > 4 ? (bytes) : 16];    \
    __shared__ __attribute__((aligned(16))) uint8_t name##5[NSLOT > 5 ? (bytes) : 16];
    RQ_RING(xr_, C::X_BYTES)
    RQ_RING(cr_, C::C_BYTES)
    RQ_RING(sr_, C::S_BYTES)
    RQ_RING(br_, C::S_BYTES)
#undef RQ_RING
    static_assert(NSLOT == 4 || NSLOT == 6, "four or six ring slots are declared");
    __shared__ __attribute__((aligned(16))) uint16_t bq0[BN * C::BLD];
    __shared__ __attribute__((aligned(16))) uint16_t bq1[BN * C::BLD];
    // DMA targets and the copies read by the dequantisation: distinct objects,
    // so the compiler never makes a read wait for the DMA in flight
    __shared__ __attribute__((aligned(16))) uint8_t sbn_s[C::SBP_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t sbn_b[C::SBP_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t sbc_s[C::SBP_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t sbc_b[C::SBP_BYTES];
#define RQ_PICK(name)                                                                   \
    [&](int u) -> uint8_t* {                                                            \
        return u == 0 ? name##0 : u == 1 ? name##1 : u == 2 ? name##2 : u == 3 ? name##3 \
             : u == 4 ? name##4 : name##5;                                              \
    }
    auto xr = RQ_PICK(xr_);
    auto cr = RQ_PICK(cr_);
    auto sr = RQ_PICK(sr_);
    auto br = RQ_PICK(br_);
#undef RQ_PICK
    auto bq = [&](int u) -> uint16_t* { return u == 0 ? bq0 : bq1; };

    const int ntiles = tiles_m * tiles_n;
    const int per_xcd = (ntiles + 7) / 8;
    const int t = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
    if (t >= ntiles) return;
    const int64_t m0 = (int64_t)(t / tiles_n) * BM, n0 = (int64_t)(t % tiles_n) * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool producer = wave >= 4;
    const int pt = tid - 256;   // producer thread index
    const int pw = wave - 4;    // producer wave index
    const int64_t runs = K >> 5, wpr = runs * BITS, G = K >> gs_shift;
    const int nst = (int)runs;

    if (producer) {
        // ---------------------------------------------------------- producers
        // Per-lane source byte offsets relative to uniform per-stage bases.
        uint32_t xoff[C::NX];
#pragma unroll
        for (int i = 0; i < C::NX; ++i) {
            const int row = (pw * C::NX + i) * 16 + (lane >> 2);
            const int chunk = (lane & 3) ^ ((row >> 2) & 3);
            int64_t grow = m0 + row;
            grow = grow < M ? grow : M - 1;
            xoff[i] = (uint32_t)((grow - m0) * K * 2 + chunk * 16);
        }
        uint32_t coff[C::NC];
#pragma unroll
        for (int i = 0; i < C::NC; ++i) {
            const int d = pt + C::NP * i;
            const int row = d / BITS;
            const int word = d - row * BITS;
            int64_t grow = n0 + (row < BN ? row : BN - 1);
            grow = grow < R ? grow : R - 1;
            coff[i] = (uint32_t)(((grow - n0) * wpr + word) * 4);
        }
        int64_t srow = n0 + (pt < BN ? pt : BN - 1);
        srow = srow < R ? srow : R - 1;
        const uint32_t soff = (uint32_t)((srow - n0) * G * C::SB);
        const uint8_t* xbase = (const uint8_t*)(x + m0 * K);
        const uint8_t* cbase = (const uint8_t*)(wq + n0 * wpr);
        const uint8_t* sbase = (const uint8_t*)scales + n0 * G * C::SB;
        const uint8_t* bbase = (const uint8_t*)biases + n0 * G * C::SB;

        auto dma = [&](int st, int slot) {
            const int64_t stc = st < nst ? st : nst - 1;  // past the end: reload the last stage
            const uint8_t* xb = xbase + stc * 64;
            const uint8_t* cb = cbase + stc * BITS * 4;
            const int64_t gb = ((stc * 32) >> gs_shift) * C::SB;
#pragma unroll
            for (int i = 0; i < C::NX; ++i)
                __builtin_amdgcn_global_load_lds((const void*)(xb + xoff[i]),
                                                 (lds_void_t*)(xr(slot) + (pw * C::NX + i) * 1024),
                                                 16, 0, 0);
#pragma unroll
            for (int i = 0; i < C::NC; ++i)
                __builtin_amdgcn_global_load_lds((const void*)(cb + coff[i]),
                                                 (lds_void_t*)(cr(slot) + (i * C::NP + pw * 64) * 4),
                                                 4, 0, 0);
            if constexpr (!SBP) {
                __builtin_amdgcn_global_load_lds((const void*)(sbase + gb + soff),
                                                 (lds_void_t*)(sr(slot) + pw * 64 * 4), C::SB, 0, 0);
                __builtin_amdgcn_global_load_lds((const void*)(bbase + gb + soff),
                                                 (lds_void_t*)(br(slot) + pw * 64 * 4), C::SB, 0, 0);
            }
        };
        // SBP: this thread's row's scales and biases of groups [8p, 8p+8)
        // are DMA'd (16 B per row each) at the start of period p-1 and copied
        // from there by the same thread at the start of period p.  Threads
        // past BN issue none.
        const int G32 = (int)G;
        auto dma_sb = [&](int period) {
            if constexpr (SBP) {
                if (pt < BN) {
                    int g0 = period * 8;
                    g0 = g0 < G32 - 8 ? g0 : G32 - 8;
                    const uint8_t* sp = (const uint8_t*)scales + (srow * G + g0) * 2;
                    const uint8_t* bp = (const uint8_t*)biases + (srow * G + g0) * 2;
                    __builtin_amdgcn_global_load_lds((const void*)sp,
                                                     (lds_void_t*)(sbn_s + pw * 64 * 16), 16, 0, 0);
                    __builtin_amdgcn_global_load_lds((const void*)bp,
                                                     (lds_void_t*)(sbn_b + pw * 64 * 16), 16, 0, 0);
                }
            }
        };
        auto dequant = [&](int slot, int bslot, int stage) {
            int local = 0;
            if constexpr (SBP) {
                const int g = (stage * 32) >> gs_shift;
                local = g & 7;
                if (((stage * 32) & ((8 << gs_shift) - 1)) == 0) {  // first stage of a period
                    if (pt < BN) {
                        const u32x4_t vs = *(const u32x4_t*)(sbn_s + pt * 16);
                        const u32x4_t vb = *(const u32x4_t*)(sbn_b + pt * 16);
                        *(u32x4_t*)(sbc_s + pt * 16) = vs;
                        *(u32x4_t*)(sbc_b + pt * 16) = vb;
                    }
                    dma_sb((g >> 3) + 1);  // after the copy has read the previous period
                }
            }
            if (pt < BN) {
                uint32_t words[BITS];
#pragma unroll
                for (int w = 0; w < BITS; ++w) words[w] = *(const uint32_t*)(cr(slot) + (pt * BITS + w) * 4);
                float s, b;
                if constexpr (SBP) {
                    const int o = pt * 16 + 2 * local;
                    s = dt_traits<SDT>::to_f32(*(const uint16_t*)(sbc_s + o));
                    b = dt_traits<SDT>::to_f32(*(const uint16_t*)(sbc_b + o));
                } else if constexpr (SDT == RQ_F32) {
                    s = *(const float*)(sr(slot) + pt * 4);
                    b = *(const float*)(br(slot) + pt * 4);
                } else {
                    s = dt_traits<SDT>::to_f32(*(const uint16_t*)(sr(slot) + pt * 4));
                    b = dt_traits<SDT>::to_f32(*(const uint16_t*)(br(slot) + pt * 4));
                }
                uint32_t d[16];
                dequant_run_fast<BITS>(words, s, b, d);
                u32x4_t* dst = (u32x4_t*)(bq(bslot) + pt * C::BLD);
#pragma unroll
                for (int q = 0; q < 4; ++q) dst[q] = u32x4_t{d[4 * q], d[4 * q + 1], d[4 * q + 2], d[4 * q + 3]};
            }
        };

        dma_sb(0);  // period 0; the wait below covers it
#pragma unroll
        for (int i = 0; i < C::AHEAD; ++i) dma(i, i);
        s_wait_vmcnt_lgkm0<(C::AHEAD - 1) * C::PER_STAGE>();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();  // barrier 0: stage 0 has landed
        asm volatile("" ::: "memory");
        dequant(0, 0, 0);
        for (int s = 0; s < nst; s += NSLOT) {
#pragma unroll
            for (int u = 0; u < NSLOT; ++u) {
                const int st = s + u;
                s_wait_vmcnt_lgkm0<(C::AHEAD - 2) * C::PER_STAGE>();
                asm volatile("" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                dma(st + C::AHEAD, (u + C::AHEAD) % NSLOT);
                if (st < nst) dequant((u + 1) % NSLOT, (u + 1) & 1, st + 1);
            }
        }
        s_wait_vmcnt_lgkm0<0>();
        return;
    }

    // -------------------------------------------------------------- consumers
    const int wm = wave >> 1, wn = wave & 1;
    const int lg = lane >> 4, lr = lane & 15;
    f32x4_t acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // LDS byte offsets of this lane's fragments (slot-relative)
    uint32_t aoff[TM];
#pragma unroll
    for (int a = 0; a < TM; ++a) {
        const int row = wm * 128 + a * 16 + lr;
        aoff[a] = (uint32_t)(row * 64 + ((lg ^ ((row >> 2) & 3)) * 16));
    }
    const uint32_t boff = (uint32_t)((wn * WN + lr) * C::BLD + lg * 8);

    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // barrier 0
    asm volatile("" ::: "memory");
    for (int s = 0; s < nst; s += NSLOT) {
#pragma unroll
        for (int u = 0; u < NSLOT; ++u) {
            const int st = s + u;
            s_wait_vmcnt_lgkm0<0>();  // own LDS reads of the previous stage are done
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (st < nst) {
                bf16x8_t af[TM], bf[TN];
#pragma unroll
                for (int a = 0; a < TM; ++a)
                    af[a] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(xr(u) + aoff[a]));
#pragma unroll
                for (int b = 0; b < TN; ++b)
                    bf[b] = __builtin_bit_cast(bf16x8_t,
                                               *(const u32x4_t*)(bq(u & 1) + boff + b * 16 * C::BLD));
#pragma unroll
                for (int a = 0; a < TM; ++a)
#pragma unroll
                    for (int b = 0; b < TN; ++b)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[a], bf[b], acc[a][b],
                                                                            0, 0, 0);
            }
        }
    }

#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int64_t n = n0 + wn * WN + b * 16 + lr;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t m = m0 + wm * 128 + a * 16 + 4 * lg + i;
                if (m < M && n < R) store_dt(y, y_dt, m * R + n, acc[a][b][i]);
            }
        }
}


// Two outputs of dtype dt (bf16 or f16) packed in one dword, RNE.
RQ_DEV uint32_t pack2_dt(int dt, float lo, float hi) {
    return dt == RQ_BF16 ? pack_bf16x2(lo, hi) : (f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16));
}

// Store one wave's 128 x WN output tile of a k64 GEMM.  The MFMAs ran with
// the weight fragment as the A operand, so lane (lg = lane / 16, lr =
// lane % 16) of 16x16 tile (a, b) holds the outputs of row a*16 + lr at
// columns b*16 + 4*lg .. +3: four consecutive columns of one row.
//  * fp32 outputs leave as one 16-byte store per tile and lane.
//  * 16-bit outputs go through a wave-private LDS strip of 16*SA rows (stg,
//    16*SA * (2*WN + 16) bytes) and leave as whole 16-byte chunks of the row
//    segment (2*WN bytes per row), instead of 2-byte scattered stores.
// Rows >= nrows and columns >= ld are not written.
template <int TM, int TN, int SA = 2>
RQ_DEV void store_wave_tile(const f32x4_t (&acc)[TM][TN], uint8_t* stg, void* __restrict__ y,
                            int y_dt, int64_t nrows, int64_t ld, int64_t r0, int64_t c0,
                            int lane) {
    constexpr int WN = TN * 16;
    const int lg = lane >> 4, lr = lane & 15;
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    if (y_dt == RQ_F32) {
        const bool vec = (((uintptr_t)y & 15) == 0) && (ld & 3) == 0;
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const int64_t m = r0 + a * 16 + lr, n = c0 + b * 16 + 4 * lg;
                if (m >= nrows) continue;
                float* dst = (float*)y + m * ld + n;
                if (vec && n + 4 <= ld) {
                    *(f32x4_t*)dst = acc[a][b];
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (n + r < ld) dst[r] = acc[a][b][r];
                }
            }
        return;
    }
    static_assert(TM % SA == 0, "whole strips of SA 16-row tiles");
    constexpr int RB = WN * 2;          // bytes per output row of the wave tile
    constexpr int SR = RB + 16;         // staging row stride (16-byte aligned)
    constexpr int CPR = RB / 16;        // 16-byte chunks per row
    constexpr int NCH = 16 * SA * CPR;  // chunks per strip of 16*SA rows
    const bool vec = (((uintptr_t)y & 15) == 0) && (ld & 7) == 0;
    uint16_t* yo = (uint16_t*)y;
#pragma unroll
    for (int a2 = 0; a2 < TM; a2 += SA) {
#pragma unroll
        for (int aa = 0; aa < SA; ++aa)
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const f32x4_t v = acc[a2 + aa][b];
                *(u32x2_t*)(stg + (aa * 16 + lr) * SR + (b * 16 + 4 * lg) * 2) =
                    u32x2_t{pack2_dt(y_dt, v[0], v[1]), pack2_dt(y_dt, v[2], v[3])};
            }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the strip is in LDS
#pragma unroll
        for (int j = 0; j < (NCH + 63) / 64; ++j) {
            const int c = lane + 64 * j;
            if (NCH % 64 != 0 && c >= NCH) break;
            const int row = c / CPR, col = c % CPR;
            const u32x4_t v = *(const u32x4_t*)(stg + row * SR + col * 16);
            const int64_t m = r0 + a2 * 16 + row, n = c0 + col * 8;
            if (m >= nrows) continue;
            if (vec && n + 8 <= ld) {
                *(u32x4_t*)(yo + m * ld + n) = v;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (n + e < ld) yo[m * ld + n + e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // strip read back before it is overwritten
    }
}

// Eight bf16 values p[0], p[stride], .., p[7 * stride] as one MFMA operand
// fragment (a column of a row-major matrix: 2-byte loads).
RQ_DEV u32x4_t gather8_bf16(const uint16_t* p, int64_t stride) {
    u32x4_t v;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        v[q] = (uint32_t)p[2 * q * stride] | ((uint32_t)p[(2 * q + 1) * stride] << 16);
    return v;
}

// The QLoRA low-rank term in the output stage: acc += scale * z . L^T for a
// wave's 128 x WN tile (rows r0.., columns c0..; acc in the weight-as-A
// layout of store_wave_tile).  z [nrows, rank] and L [ncols, rank] are bf16
// and small (rank <= 64), read straight from global memory: lane (lg, lr)
// takes elements 8*lg .. +7 of a 32-wide rank slice of row lr of each 16-row
// tile; slices past the rank and rows past the bounds read as zero.  With
// lo.stored, L comes as its transpose [rank, l_ld] (eight 2-byte loads a
// fragment, once per tile).
template <int TM, int TN>
RQ_DEV void lora_epilogue(f32x4_t (&acc)[TM][TN], const rq::LoraArgs& lo, int64_t nrows,
                          int64_t ncols, int64_t r0, int64_t c0, int lane) {
    const int lg = lane >> 4, lr = lane & 15;
    const uint16_t* z = (const uint16_t*)lo.z;
    const uint16_t* l = (const uint16_t*)lo.l;
    for (int j0 = 0; j0 < lo.rank; j0 += 32) {
        const int j = j0 + 8 * lg;
        const bool has = j < lo.rank;
        bf16x8_t zf[TM], lf[TN];
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            const int64_t m = r0 + a * 16 + lr;
            u32x4_t v = {0u, 0u, 0u, 0u};
            if (has && m < nrows) v = *(const u32x4_t*)(z + m * lo.rank + j);
            zf[a] = __builtin_bit_cast(bf16x8_t, v);
        }
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int64_t n = c0 + b * 16 + lr;
            u32x4_t v = {0u, 0u, 0u, 0u};
            if (has && n < ncols)
                v = lo.stored ? gather8_bf16(l + j * lo.l_ld + n, lo.l_ld)
                              : *(const u32x4_t*)(l + n * lo.rank + j);
            lf[b] = __builtin_bit_cast(bf16x8_t, v);
        }
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b) {
                const f32x4_t t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    lf[b], zf[a], f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[a][b][r] = fmaf(lo.scale, t[r], acc[a][b][r]);
            }
    }
}

// The fused QLoRA layer's down-projection, computed in the GEMM (rank 16).
// Each MFMA wave of a (wm) pair accumulated z over the k-steps h == wn of
// every stage (accz: lane (lg, lr) holds row lr of 16-row tile a, ranks
// 4 lg .. +3) from the activation fragments of its main MFMAs.  Once the
// ring slots are free (a barrier every wave of the block joins), the pair's
// fp32 partials are exchanged through one slot (zx: [4 waves][rows][16]),
// summed in the same order by both waves, rounded once to bf16, stored to
// z_out by the column-tile-0 blocks (one wave of the pair), and the term
// scale * z . L^T is added to acc (L [ncols, 16] bf16 from global memory,
// or its transpose [16, l_ld] when lo.stored).
template <int TM, int TN>
RQ_DEV void fused_lora_tail(f32x4_t (&acc)[TM][TN], const f32x4_t (&accz)[TM], float* zx, int wm,
                            int wn, int lane, const rq::LoraArgs& lo, bool write_z, int64_t nrows,
                            int64_t ncols, int64_t r0, int64_t c0) {
    const int lg = lane >> 4, lr = lane & 15;
    constexpr int ROWS = TM * 16;
    // L's fragments first: their global-memory latency overlaps the exchange
    const uint16_t* l = (const uint16_t*)lo.l;
    bf16x8_t lf[TN];
#pragma unroll
    for (int b = 0; b < TN; ++b) {
        const int64_t n = c0 + b * 16 + lr;
        u32x4_t v = {0u, 0u, 0u, 0u};
        if (lg < 2 && n < ncols)
            v = lo.stored ? gather8_bf16(l + 8 * lg * lo.l_ld + n, lo.l_ld)
                          : *(const u32x4_t*)(l + n * 16 + 8 * lg);
        lf[b] = __builtin_bit_cast(bf16x8_t, v);
    }
#pragma unroll
    for (int a = 0; a < TM; ++a)
        *(f32x4_t*)(zx + ((wm * 2 + wn) * ROWS + a * 16 + lr) * 16 + 4 * lg) = accz[a];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the partials are in LDS
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();        // the pair's partials are visible (every wave joins)
    asm volatile("" ::: "memory");
    bf16x8_t zf[TM];
#pragma unroll
    for (int a = 0; a < TM; ++a) {
        u32x4_t v = {0u, 0u, 0u, 0u};
        if (lg < 2) {
            const float* p0 = zx + ((wm * 2) * ROWS + a * 16 + lr) * 16 + 8 * lg;
            const float* p1 = p0 + ROWS * 16;
            const f32x4_t a0 = *(const f32x4_t*)p0, a1 = *(const f32x4_t*)(p0 + 4);
            const f32x4_t b0 = *(const f32x4_t*)p1, b1 = *(const f32x4_t*)(p1 + 4);
            v = u32x4_t{pack_bf16x2(a0[0] + b0[0], a0[1] + b0[1]),
                        pack_bf16x2(a0[2] + b0[2], a0[3] + b0[3]),
                        pack_bf16x2(a1[0] + b1[0], a1[1] + b1[1]),
                        pack_bf16x2(a1[2] + b1[2], a1[3] + b1[3])};
            const int64_t m = r0 + a * 16 + lr;
            if (write_z && m < nrows) *(u32x4_t*)((uint16_t*)lo.z_out + m * 16 + 8 * lg) = v;
        }
        zf[a] = __builtin_bit_cast(bf16x8_t, v);
    }
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const f32x4_t t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                lf[b], zf[a], f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[a][b][r] = fmaf(lo.scale, t[r], acc[a][b][r]);
        }
}

// A producer's 16-byte chunk of 8 activations for a bf16 LDS tile.  bf16
// activations load it as is; fp32 ones (XF) load 32 bytes and round them to
// bf16 (RNE) when the chunk is stored, so the tile, the MFMA operands and
// everything after them are the same for both.
template <bool XF>
struct XChunk {
    static constexpr int EB = XF ? 4 : 2;  // bytes per activation element
    typedef const __attribute__((address_space(1))) u32x4_t* gv_t;
    u32x4_t v[XF ? 2 : 1];
    RQ_DEV void load(const uint8_t* p) {
        v[0] = *(gv_t)p;
        if constexpr (XF) v[1] = *((gv_t)p + 1);
    }
    RQ_DEV u32x4_t bf16() const {
        if constexpr (XF) {
            return u32x4_t{pack_bf16x2(__uint_as_float(v[0][0]), __uint_as_float(v[0][1])),
                           pack_bf16x2(__uint_as_float(v[0][2]), __uint_as_float(v[0][3])),
                           pack_bf16x2(__uint_as_float(v[1][0]), __uint_as_float(v[1][1])),
                           pack_bf16x2(__uint_as_float(v[1][2]), __uint_as_float(v[1][3]))};
        } else {
            return v[0];
        }
    }
};

// ------------------------------------------------------------- qmm_t_k64
//
// The warp-specialised GEMM with 64-element contraction stages (bf16
// activations, M >= 256, 16-bit scales, K a multiple of 8 groups).  The
// per-CU memory rate of these kernels is set by how many L2 requests a CU
// keeps in flight, so every request here carries a whole 128-byte line: a
// producer wave-load covers 8 activation rows x 128 B, a weight row's codes
// for a stage are 64 contiguous codes, and each row's (scale, bias) values
// arrive 8 groups per 16-byte load, once per 8 groups.  Waves 0-3 run MFMAs
// (2x2, wave tile 128 x BN/2, two k-steps of 32 per stage); waves 4-7 keep
// D stages of loads in flight in registers, write the activations to a
// 2-slot LDS ring (16-byte chunks XOR-swizzled by row) and dequantize the
// stage's codes straight from registers into a 2-slot bf16 ring (128-byte
// rows, the same chunk swizzle; a padded 144-byte row measured 1-6 %
// slower).  One
// barrier per stage.
//  * A wave64 VALU op costs ~6-8 cycles and runs beside the MFMA wave on
//    the same SIMD, so the dequantization is split evenly over all 256
//    producer lanes: each takes NJ jobs of JW packed words (one 8-code word
//    at 4 bits with BN = 160, one 32-code run otherwise), reading the job's
//    fp32 (scale, bias) from an LDS table that one thread per row refreshes
//    once per 8 groups.
//  * The MFMA waves hold 160 accumulator registers, so their fragments are
//    software-pipelined by hand (B fragments of the next k-step and A
//    fragments two MFMA groups ahead), with scheduling barriers keeping the
//    order: the compiler's own order waited on every fragment read.
template <int BITS, int SDT, int BN, int GSH, int BM, bool FZ = false, bool XF = false>
__global__ __launch_bounds__(kWsBlock, 1) void qmm_t_k64(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, int64_t M, int64_t R, int64_t K, void* __restrict__ y,
    int y_dt, int tiles_m, int tiles_n, rq::LoraArgs lora, int splits, float* __restrict__ part) {
    static_assert(BM == 256 || BM == 128 || BM == 64, "block rows");
    constexpr int WN = BN / 2;
    constexpr int TM = BM / 32, TN = WN / 16;   // 16x16 MFMA tiles per wave (2x2 waves)
    constexpr int XL = BM / 32;                 // activation loads per producer lane per stage
    constexpr int BLD = 64;                  // bf16 ring row: 8 chunks of 16 B, XOR-swizzled by row & 7
    constexpr int D = RQ_K64_DEPTH;          // stages of loads in flight per producer thread
    constexpr int P = (8 << GSH) / 64;       // stages per 8-group (scale, bias) chunk: 4, 8, 16
    static_assert(P % D == 0, "the register ring index is the unrolled stage index mod D");
    static_assert(SDT != RQ_F32, "16-bit scales");
    static_assert(BN <= 256, "one producer thread stages one row's (scale, bias)");
    // SB stages per barrier: a small tile's stage is short next to the fixed
    // cost of the barrier and the LDS round trip around it, so its producers
    // stage SB stages into a 2 SB-slot ring before each barrier and its MFMA
    // waves run all SB of them after it
    constexpr int SB = BM == 64 ? RQ_K64_SB64 : ((BM == 128 && BN <= 128 && !FZ) ? RQ_K64_SB128 : 1);
    constexpr int NS = 2 * SB;  // ring slots
    static_assert(P % SB == 0 && (SB == 1 || SB == 2), "whole groups of stages per period");
    __shared__ __attribute__((aligned(16))) uint8_t xsr[NS][BM * 128];
    __shared__ __attribute__((aligned(16))) uint16_t bqr[NS][BN * BLD];
    __shared__ __attribute__((aligned(16))) float sbf[2][BN * 16];  // fp32 (scale, bias), [row][8 groups]
    uint8_t* const xs0 = xsr[0];
    uint8_t* const xs1 = xsr[1];

    // split-K (splits > 1): block tt is tile tt % ntiles over the ks = tt / ntiles-th
    // share of the contraction, whole 8-group periods each, written as an fp32
    // partial tile to part[ks] (an XCD's contiguous run of blocks then shares
    // one K range: the same activation and weight panels in its L2)
    const int ntiles = tiles_m * tiles_n;
    const int nblk = ntiles * splits;
    const int per_xcd = (nblk + 7) / 8;
    const int tt = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
    if (tt >= nblk) return;
    const int ks = tt / ntiles, t = tt - ks * ntiles;
    int mt, nt;
    k64_tile(t, tiles_m, tiles_n, mt, nt);
    const int64_t m0 = (int64_t)mt * BM, n0 = (int64_t)nt * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t wpr = (K >> 5) * BITS, G = K >> GSH;
    // this block's periods [pb, pe) of the contraction (all of them unsplit)
    const int nper_all = (int)((K >> 6) / P);
    const int pb = (int)((int64_t)ks * nper_all / splits), pe = (int)((int64_t)(ks + 1) * nper_all / splits);
    const int nst = splits > 1 ? (pe - pb) * P : (int)(K >> 6);
    const int nper = (nst + P - 1) / P;
    const int64_t st0 = (int64_t)pb * P;  // first stage
    if (nst <= 0) return;

    constexpr int SW = 2 * BITS;                              // packed words per row per stage
    constexpr int JW = (BITS == 4 && (BN == 160 || BN == 96)) ? 1 : BITS;  // words per dequant job
    constexpr int JPR = SW / JW;                              // jobs per row per stage
    constexpr int NJ = BN * JPR / 256;                        // jobs per producer thread
    constexpr int JC = 32 * JW / BITS;                        // codes per job
    static_assert(NJ * 256 == BN * JPR, "every producer thread gets the same dequant work");

    if (wave >= 4) {
        // ---------------------------------------------------------- producers
        if (RQ_K64_PPRIO) __builtin_amdgcn_s_setprio(RQ_K64_PPRIO);
        const int pt = tid - 256, pw = wave - 4;
        typedef const __attribute__((address_space(1))) u32x4_t* gv_t;
        typedef const __attribute__((address_space(1))) uint32_t* gw_t;
        uint32_t xoff[XL], xdst[XL];
#pragma unroll
        for (int i = 0; i < XL; ++i) {
            const int row = (pw * XL + i) * 8 + (lane >> 3);
            const int chunk = lane & 7;
            int64_t grow = m0 + row;
            grow = grow < M ? grow : M - 1;
            xoff[i] = (uint32_t)((grow - m0) * K * XChunk<XF>::EB + chunk * 8 * XChunk<XF>::EB);
            xdst[i] = (uint32_t)(row * 128 + ((chunk ^ (row & 7)) * 16));
        }
        const uint8_t* xbase = (const uint8_t*)x + (m0 * K + st0 * 64) * XChunk<XF>::EB;
        // dequant jobs: job j = pt + 256 i is part j % JPR (JW words) of tile row j / JPR
        const uint32_t* wtile = wq + n0 * wpr + st0 * SW;
        uint32_t coff[NJ], qoff[NJ], soff[NJ], qc0[NJ];
#pragma unroll
        for (int i = 0; i < NJ; ++i) {
            const int j = pt + 256 * i, row = j / JPR, part = j % JPR;
            const int rr = n0 + row < R ? row : (int)(R - 1 - n0);
            coff[i] = (uint32_t)(rr * wpr + part * JW);
            qoff[i] = (uint32_t)(row * BLD);
            qc0[i] = (uint32_t)((part * (JC / 8)) | ((row & 7) << 8));  // first chunk, row key
            soff[i] = (uint32_t)(row * 16 + (GSH == 5 ? 2 * ((part * JC) >> 5) : 0));
        }
        // (scale, bias) staging: thread pt < BN converts row pt's 8 groups of a period
        const bool has_row = pt < BN;
        int64_t wrow = n0 + (has_row ? pt : 0);
        wrow = wrow < R ? wrow : R - 1;
        const int64_t g_base = (st0 * 64) >> GSH;  // the range's first group
        const uint16_t* srow_p = (const uint16_t*)scales + wrow * G + g_base;
        const uint16_t* brow_p = (const uint16_t*)biases + wrow * G + g_base;
        const int g_rem = (int)(G - g_base);  // groups of the row from there

        XChunk<XF> xv[D][XL];
        uint32_t cv[D][NJ][JW];
        auto issue = [&](int st, int r) {
            const int sc = st < nst ? st : nst - 1;
            const uint8_t* xb = xbase + (int64_t)sc * 64 * XChunk<XF>::EB;
#pragma unroll
            for (int i = 0; i < XL; ++i) xv[r][i].load(xb + xoff[i]);
            const uint32_t* ws = wtile + (int64_t)sc * SW;
#pragma unroll
            for (int i = 0; i < NJ; ++i) {
                if constexpr (JW % 4 == 0) {
#pragma unroll
                    for (int q = 0; q < JW / 4; ++q) {
                        const u32x4_t v = *((gv_t)(ws + coff[i]) + q);
                        cv[r][i][4 * q] = v[0]; cv[r][i][4 * q + 1] = v[1];
                        cv[r][i][4 * q + 2] = v[2]; cv[r][i][4 * q + 3] = v[3];
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < JW; ++q) cv[r][i][q] = *((gw_t)(ws + coff[i]) + q);
                }
            }
        };
        u32x4_t s_nxt = {0u, 0u, 0u, 0u}, b_nxt = s_nxt;
        auto load_sb = [&](int per) {
            int g0 = per * 8;
            g0 = g0 < g_rem - 8 ? g0 : g_rem - 8;  // past the row: an unused reload
            if (has_row) {
                s_nxt = *(gv_t)(srow_p + g0);
                b_nxt = *(gv_t)(brow_p + g0);
            }
        };
        auto put_sb = [&](int buf) {
            if (has_row) {
                float* d = sbf[buf] + pt * 16;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t sw = s_nxt[q], bw = b_nxt[q];
                    *(f32x4_t*)(d + 4 * q) = f32x4_t{
                        dt_traits<SDT>::to_f32((uint16_t)(sw & 0xffffu)),
                        dt_traits<SDT>::to_f32((uint16_t)(bw & 0xffffu)),
                        dt_traits<SDT>::to_f32((uint16_t)(sw >> 16)),
                        dt_traits<SDT>::to_f32((uint16_t)(bw >> 16))};
                }
            }
        };
        load_sb(0);
        put_sb(0);
        load_sb(1);
#pragma unroll
        for (int r = 0; r < D; ++r) issue(r, r);
        __builtin_amdgcn_s_waitcnt(0xc07f);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();  // period 0's (scale, bias) are staged
        asm volatile("" ::: "memory");

        for (int per = 0; per < nper; ++per) {
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int st = per * P + u;
                uint8_t* xs = xsr[u % NS];
                uint16_t* bq = bqr[u % NS];
                if (u == 0) {
                    put_sb((per + 1) & 1);  // the next period's values (read from stage (per+1)*P on)
                    load_sb(per + 2);
                }
#pragma unroll
                for (int i = 0; i < XL; ++i) *(u32x4_t*)(xs + xdst[i]) = xv[u % D][i].bf16();
                const float* sb = sbf[per & 1] + 2 * ((u * 64) >> GSH);
#pragma unroll
                for (int i = 0; i < NJ; ++i) {
                    typedef float f32x2_t __attribute__((ext_vector_type(2)));
                    const f32x2_t sv = *(const f32x2_t*)(sb + soff[i]);
                    uint32_t d[JC / 2];
                    if constexpr (JW == 1) {
                        dequant_word4(cv[u % D][i][0], sv[0], sv[1], d);
                    } else {
                        dequant_run_fast<BITS>(cv[u % D][i], sv[0], sv[1], d);
                    }
                    u32x4_t* dst = (u32x4_t*)(bq + qoff[i]);
#pragma unroll
                    for (int q = 0; q < JC / 8; ++q)
                        dst[((qc0[i] & 0xff) + q) ^ (qc0[i] >> 8)] =
                            u32x4_t{d[4 * q], d[4 * q + 1], d[4 * q + 2], d[4 * q + 3]};
                }
                issue(st + D, u % D);
                if (u % SB == SB - 1) {
                    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): these stages' LDS writes are done
                    asm volatile("" ::: "memory");
                    __builtin_amdgcn_s_barrier();
                    asm volatile("" ::: "memory");
                }
            }
        }
        if constexpr (FZ) {
            // the MFMA waves' two barriers of the down-projection exchange
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
        }
        return;
    }

    // -------------------------------------------------------------- consumers
    if (RQ_K64_CPRIO) __builtin_amdgcn_s_setprio(RQ_K64_CPRIO);
    const int wm = wave >> 1, wn = wave & 1;
    const int lg = lane >> 4, lr = lane & 15;
    f32x4_t acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    uint32_t aoff[2][TM];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            const int row = wm * (BM / 2) + a * 16 + lr;
            aoff[h][a] = (uint32_t)(row * 128 + (((h * 4 + lg) ^ (row & 7)) * 16));
        }
    // B fragment rows wn*WN + 16 b + lr all have key lr & 7 (WN % 8 == 0)
    static_assert(WN % 8 == 0, "a fragment row's swizzle key is lr & 7");
    uint32_t boff[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
        boff[h] = (uint32_t)((wn * WN + lr) * BLD + (((h * 4 + lg) ^ (lr & 7)) * 8));
    // fused down-projection: this wave's 16 x 32 fragment of a (rank lr,
    // columns 8 lg .. +7 of k-step h == wn) for the current and next stage
    f32x4_t accz[TM];
    u32x4_t zfa_cur = {0u, 0u, 0u, 0u}, zfa_nxt = zfa_cur;
    const uint16_t* zarow = nullptr;
    // wn as a wave-uniform (scalar) value selects the main loop's
    // instantiation (an EXEC-masked MFMA would still run)
    const int wn_s = __builtin_amdgcn_readfirstlane(wn);
    if constexpr (FZ) {
#pragma unroll
        for (int a = 0; a < TM; ++a) accz[a] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        zarow = (const uint16_t*)lora.a + (int64_t)lr * lora.a_ld + 32 * wn + 8 * lg;
        zfa_nxt = *(const u32x4_t*)zarow;
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // the producers' prologue barrier
    asm volatile("" ::: "memory");

    // the main loop, instantiated once per value of wn in the fused form so
    // that the k-step a wave projects (h == ZH) is fixed at compile time:
    // no branch inside the MFMA schedule
    auto main_loop = [&](auto zh_c) {
        constexpr int ZH = decltype(zh_c)::value;
        for (int per = 0; per < nper; ++per) {
#pragma unroll
            for (int u = 0; u < P; ++u) {
                const int st = per * P + u;
                if (u % SB == 0) {
                    __builtin_amdgcn_s_waitcnt(0xc07f);  // own LDS reads of the previous stages are done
                    asm volatile("" ::: "memory");
                    __builtin_amdgcn_s_barrier();
                    asm volatile("" ::: "memory");
                }
                if (st < nst) {
                    const uint8_t* xs = xsr[u % NS];
                    const uint16_t* bq = bqr[u % NS];
                    if constexpr (FZ) {
                        zfa_cur = zfa_nxt;
                        if (st + 1 < nst) zfa_nxt = *(const u32x4_t*)(zarow + (int64_t)(st + 1) * 64);
                    }
                    // software pipeline over (h, a): B fragments of k-step h+1 are read
                    // while k-step h runs; A fragments rotate through 3 registers, read
                    // 2 MFMA groups (10 MFMAs) ahead of their use.
                    bf16x8_t bf[2][TN], af[3];
                    auto rdA = [&](int h, int a) {
                        return __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(xs + aoff[h][a]));
                    };
                    auto rdB = [&](int h, int b) {
                        return __builtin_bit_cast(bf16x8_t,
                                                  *(const u32x4_t*)(bq + boff[h] + b * 16 * BLD));
                    };
#pragma unroll
                    for (int b = 0; b < TN; ++b) bf[0][b] = rdB(0, b);
                    af[0] = rdA(0, 0);
                    af[1] = rdA(0, 1);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
#pragma unroll
                        for (int a = 0; a < TM; ++a) {
                            const int q = h * TM + a + 2;   // the (h, a) index read now
                            if (q < 2 * TM) af[q % 3] = rdA(q / TM, q % TM);
                            if (h == 0 && a == (TM > 2 ? 2 : TM - 1)) {
#pragma unroll
                                for (int b = 0; b < TN; ++b) bf[1][b] = rdB(1, b);
                            }
                            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                            for (int b = 0; b < TN; ++b)
                                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                    bf[h][b], af[(h * TM + a) % 3], acc[a][b], 0, 0, 0);
                            if constexpr (FZ) {
                                if (h == ZH)  // folds: h and ZH are both constants here
                                    accz[a] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                        __builtin_bit_cast(bf16x8_t, zfa_cur), af[(h * TM + a) % 3],
                                        accz[a], 0, 0, 0);
                            }
                            __builtin_amdgcn_sched_barrier(0);
                        }
                    }
                }
            }
        }
    };
    if (FZ && wn_s != 0)
        main_loop(std::integral_constant<int, 1>{});
    else
        main_loop(std::integral_constant<int, 0>{});

    // after the last barrier the ring slot of stage nst - 2 SB (nst % NS: nst
    // is a whole number of periods) is read by nobody and written by nobody:
    // 8 KB of it per wave stage the output
    if constexpr (FZ) {
        __builtin_amdgcn_s_waitcnt(0xc07f);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();  // every wave is done with both ring slots
        asm volatile("" ::: "memory");
        fused_lora_tail<TM, TN>(acc, accz, (float*)((nst & 1) ? xs0 : xs1), wm, wn, lane, lora,
                                lora.z_out != nullptr && nt == 0 && wn == 0, M, R,
                                m0 + wm * (BM / 2), n0 + wn * WN);
    } else if (lora.z) {
        lora_epilogue<TM, TN>(acc, lora, M, R, m0 + wm * (BM / 2), n0 + wn * WN, lane);
    }
    // strips of 32 rows (BM 256: 8 KB of the free slot per wave) or 16 (BM 128: 4 KB)
    constexpr int SA = BM == 256 ? 2 : 1;
    static_assert(16 * SA * (BN + 16) <= BM * 32, "a wave's staging strip fits its share of a slot");
    if (splits > 1)  // fp32 partial tile of split ks
        store_wave_tile<TM, TN, SA>(acc, xsr[nst % NS] + wave * (BM * 32),
                                    part + (int64_t)ks * M * R, RQ_F32, M, R, m0 + wm * (BM / 2),
                                    n0 + wn * WN, lane);
    else
        store_wave_tile<TM, TN, SA>(acc, xsr[nst % NS] + wave * (BM * 32), y, y_dt, M,
                                    R, m0 + wm * (BM / 2), n0 + wn * WN, lane);
}


// ------------------------------------------------------------- qmm_n_k64
//
// Transposed product dX[M, K] = dY[M, R] . W^[R, K] (the QLoRA backward),
// warp-specialised like qmm_t_k64: block tile 256 (dY rows) x 128 (output
// columns k), 64 weight rows r per stage.  The contraction runs over r, the
// rows of W, while the packed codes run along k, so the weight operand needs
// a transpose somewhere.  It happens in the MFMA waves' fragment reads:
//  * producers (waves 4-7) dequantize exactly like qmm_t_k64's: each thread
//    takes one 32-code run of one weight row per stage (row pt % 64, run
//    pt / 64 of the tile's four), its codes and (scale, bias) loaded straight
//    into registers D stages ahead, and writes the 32 bf16 values as two
//    16-byte stores of the natural [r][k] tile (k contiguous, 256-byte rows);
//    they also write the dY tile (256 rows x 128 B) to a 2-slot ring;
//  * MFMA waves (0-3) read each weight fragment (8 consecutive r of one k
//    column per lane) with two gfx950 ds_read_b64_tr_b16: within 16 lanes,
//    source lane 4s + a reads 4 columns 4a .. 4a+3 of row s and result lane
//    4a + b receives column 4a + b of rows 0..3.
// The [r][k] tile's 16-byte chunks are XOR-swizzled by nkey(r): a bijection
// on r % 8, so the 8 rows of a producer store group hit 8 bank groups, whose
// upper two bits are a bijection on each aligned quad of rows, so the 4 rows x
// 2 chunks of a 16-lane transposed read hit 8.  No code tile is staged in
// LDS and no (scale, bias) table: the producers' critical path has no LDS
// read, and the tile is written with half as many stores as the earlier
// r-contiguous layout needed.
// BN = 160 (4- and 8-bit codes, K % 160 == 0): the 2560-wide outputs of
// the 2.9B shapes are 16 x 16 = 256 tiles (one round on 256 CUs) instead of
// 16 x 20 = 320 at BN = 128.  A stage row is 20 chunks of 8 codes; producer
// thread (row, q) dequantizes chunks 5q .. 5q+4 (40 codes, at most three
// groups: their (scale, bias) values are loaded per stage), and tile rows are
// padded to 24 chunks so that the swizzle stays inside aligned 8-chunk
// groups.
// Requires 16-bit scales, R % 64 == 0 and K % BN == 0.
RQ_DEV int nkey(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }
// physical 16-byte chunk of chunk c in tile row r
RQ_DEV int nchunk(int c, int r) { return (c & ~7) | ((c ^ nkey(r)) & 7); }

template <int BITS, int SDT, int BN = 128, bool FZ = false, bool XF = false>
__global__ __launch_bounds__(kWsBlock, 1) void qmm_n_k64(
    const void* __restrict__ x, const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, int64_t M, int64_t R, int64_t K, int gs_shift,
    void* __restrict__ y, int y_dt, int tiles_m, int tiles_n, rq::LoraArgs lora) {
    constexpr int BM = 256, WN = BN / 2;
    constexpr int TM = 8, TN = WN / 16;
    constexpr int D = 2;  // stages of loads in flight per producer thread: the ring slot index
    constexpr int ROWB = BN == 160 ? 384 : BN * 2;  // bytes per row of the bf16 weight tile
    static_assert(SDT != RQ_F32, "16-bit scales");
    static_assert(BN == 128 || (BN == 160 && (BITS == 4 || BITS == 8) && !FZ), "tile width");
    __shared__ __attribute__((aligned(16))) uint8_t xs0[BM * 128];
    __shared__ __attribute__((aligned(16))) uint8_t xs1[BM * 128];
    __shared__ __attribute__((aligned(16))) uint8_t bq0[64 * ROWB];
    __shared__ __attribute__((aligned(16))) uint8_t bq1[64 * ROWB];
    // fused form with the adapter as stored (B [R, 16]): a stage's 64 rows of
    // B, 2 KB, copied as they lie by the first two producer waves
    __shared__ __attribute__((aligned(16))) uint8_t zb[2][FZ ? 64 * 32 : 16];

    const int ntiles = tiles_m * tiles_n;
    const int per_xcd = (ntiles + 7) / 8;
    const int t = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
    if (t >= ntiles) return;
    const int64_t m0 = (int64_t)(t / tiles_n) * BM, k0 = (int64_t)(t % tiles_n) * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t wpr = (K >> 5) * BITS, G = K >> gs_shift;
    const int nst = (int)(R >> 6);

    if (wave >= 4) {
        // ---------------------------------------------------------- producers
        if (RQ_K64_PPRIO) __builtin_amdgcn_s_setprio(RQ_K64_PPRIO);
        const int pt = tid - 256, pw = wave - 4;
        typedef const __attribute__((address_space(1))) u32x4_t* gv_t;
        typedef const __attribute__((address_space(1))) uint32_t* gw_t;
        typedef const __attribute__((address_space(1))) uint16_t* gh_t;
        uint32_t xoff[8], xdst[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int row = (pw * 8 + i) * 8 + (lane >> 3);
            const int chunk = lane & 7;
            int64_t grow = m0 + row;
            grow = grow < M ? grow : M - 1;
            xoff[i] = (uint32_t)((grow - m0) * R * XChunk<XF>::EB + chunk * 8 * XChunk<XF>::EB);
            xdst[i] = (uint32_t)(row * 128 + ((chunk ^ (row & 7)) * 16));
        }
        const uint8_t* xbase = (const uint8_t*)x + m0 * R * XChunk<XF>::EB;
        if constexpr (BN == 160) {
            // Lane L of producer wave pw takes row jr = 16 pw + L / 4 of each
            // stage and its chunks 5 q .. 5 q + 4 (q = L % 4, 8 codes each), so
            // one code-load instruction covers 16 rows' contiguous 80 B.  A
            // row's (scale, bias) values of the tile's groups (at most 4 from
            // g0, 6 at gs 32) are loaded once per lane quad -- lane q takes
            // group g0 + q, and g0 + 4 + q at gs 32 -- and handed to the lanes
            // that need them with ds_bpermute (a lane's 40 codes touch at most
            // two groups, three at gs 32).
            constexpr int NC = 5, WPC = BITS / 4, NG = 3;
            typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
            const int jq = lane & 3, jr = pw * 16 + (lane >> 2);
            const uint32_t* wbase = wq + ((k0 >> 3) + NC * jq) * WPC;
            const int64_t kc0 = k0 + 8 * NC * jq;
            const int64_t g0 = k0 >> gs_shift;                // the tile's first group
            const int rel0 = (int)((kc0 >> gs_shift) - g0);  // this lane's first group, from g0
            const bool g32 = gs_shift == 5;
            int gsel[NC];
            uint32_t qdst[NC];
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                gsel[i] = (int)(((kc0 + 8 * i) >> gs_shift) - (kc0 >> gs_shift));
                qdst[i] = (uint32_t)(jr * ROWB + (nchunk(NC * jq + i, jr) << 4));
            }
            // the groups this lane loads, clamped inside the row (past-the-row
            // ones are never selected)
            const int ga = g0 + jq < G ? jq : (int)(G - 1 - g0);
            const int gb = g0 + 4 + jq < G ? 4 + jq : (int)(G - 1 - g0);
            const uint16_t* sbase = (const uint16_t*)scales + g0;
            const uint16_t* bbase = (const uint16_t*)biases + g0;
            int srcl[NG], slot[NG];  // bpermute byte address and load slot of pairs rel0 + j
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                const int rel = rel0 + j;
                srcl[j] = ((lane & ~3) | (rel & 3)) * 4;
                slot[j] = rel >> 2;
            }
            XChunk<XF> xv[D][8];
            uint32_t cv[D][NC * WPC];
            uint32_t sv[D][2];  // scale | bias << 16 of groups g0 + jq and g0 + 4 + jq
            auto issue = [&](int st, int r) {
                const int sc = st < nst ? st : nst - 1;
                const uint8_t* xb = xbase + (int64_t)sc * 64 * XChunk<XF>::EB;
#pragma unroll
                for (int i = 0; i < 8; ++i) xv[r][i].load(xb + xoff[i]);
                const int64_t row = (int64_t)sc * 64 + jr;
                const uint32_t* ws = wbase + row * wpr;
                if constexpr (WPC == 1) {
#pragma unroll
                    for (int q = 0; q < NC; ++q) cv[r][q] = *((gw_t)ws + q);
                } else {
                    typedef const __attribute__((address_space(1))) u32x2_t* g2_t;
#pragma unroll
                    for (int q = 0; q < NC; ++q) {
                        const u32x2_t v = *((g2_t)ws + q);
                        cv[r][2 * q] = v[0];
                        cv[r][2 * q + 1] = v[1];
                    }
                }
                sv[r][0] = (uint32_t)*(gh_t)(sbase + row * G + ga) |
                           ((uint32_t)*(gh_t)(bbase + row * G + ga) << 16);
                if (g32)
                    sv[r][1] = (uint32_t)*(gh_t)(sbase + row * G + gb) |
                               ((uint32_t)*(gh_t)(bbase + row * G + gb) << 16);
            };
#pragma unroll
            for (int r = 0; r < D; ++r) issue(r, r);
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();  // pairs with the MFMA waves' first barrier
            asm volatile("" ::: "memory");
            for (int s0 = 0; s0 < nst; s0 += 2) {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int st = s0 + u;
                    uint8_t* xs = u ? xs1 : xs0;
                    uint8_t* bq = u ? bq1 : bq0;
#pragma unroll
                    for (int i = 0; i < 8; ++i) *(u32x4_t*)(xs + xdst[i]) = xv[u][i].bf16();
                    float sf[NG], bf[NG];
#pragma unroll
                    for (int j = 0; j < NG; ++j) {
                        uint32_t pr = 0u;
                        if (j < 2 || g32) {
                            pr = (uint32_t)__builtin_amdgcn_ds_bpermute(srcl[j], (int)sv[u][0]);
                            if (g32) {
                                const uint32_t p1 =
                                    (uint32_t)__builtin_amdgcn_ds_bpermute(srcl[j], (int)sv[u][1]);
                                pr = slot[j] ? p1 : pr;
                            }
                        }
                        sf[j] = dt_traits<SDT>::to_f32((uint16_t)(pr & 0xffffu));
                        bf[j] = dt_traits<SDT>::to_f32((uint16_t)(pr >> 16));
                    }
#pragma unroll
                    for (int i = 0; i < NC; ++i) {
                        const float sc = gsel[i] == 0 ? sf[0] : (gsel[i] == 1 ? sf[1] : sf[2]);
                        const float bc = gsel[i] == 0 ? bf[0] : (gsel[i] == 1 ? bf[1] : bf[2]);
                        uint32_t d[4];
                        if constexpr (WPC == 1) {
                            // byte converts here: the fp8 pair conversion of dequant_word4
                            // measured 3-4 % slower in this kernel ([8192, 2048] at M = 4096)
                            uint32_t lo = cv[u][i] & 0x0F0F0F0Fu;         // codes 0, 2, 4, 6
                            uint32_t hi = (cv[u][i] >> 4) & 0x0F0F0F0Fu;  // codes 1, 3, 5, 7
                            asm("" : "+v"(lo));
                            asm("" : "+v"(hi));
#pragma unroll
                            for (int k = 0; k < 4; ++k)
                                d[k] = pack_bf16x2(fmaf(sc, (float)(uint8_t)(lo >> (8 * k)), bc),
                                                   fmaf(sc, (float)(uint8_t)(hi >> (8 * k)), bc));
                        } else {
#pragma unroll
                            for (int w = 0; w < 2; ++w) {
                                uint32_t v = cv[u][2 * i + w];
                                asm("" : "+v"(v));
#pragma unroll
                                for (int k = 0; k < 2; ++k)
                                    d[2 * w + k] =
                                        pack_bf16x2(fmaf(sc, (float)(uint8_t)(v >> (16 * k)), bc),
                                                    fmaf(sc, (float)(uint8_t)(v >> (16 * k + 8)), bc));
                            }
                        }
                        *(u32x4_t*)(bq + qdst[i]) = u32x4_t{d[0], d[1], d[2], d[3]};
                    }
                    issue(st + D, u);
                    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this stage's LDS writes are done
                    asm volatile("" ::: "memory");
                    __builtin_amdgcn_s_barrier();
                    asm volatile("" ::: "memory");
                }
            }
            return;
        }
        // the dequantization job: run jq of row jr of each stage; the four
        // runs of a row go to one lane quad (16 rows per wave), so one code
        // load covers 16 rows' contiguous 64 B
        const int jr = pw * 16 + (lane >> 2), jq = lane & 3;
        const uint32_t* wbase = wq + (k0 >> 5) * BITS + jq * BITS;
        const int64_t gidx = (k0 + jq * 32) >> gs_shift;
        const uint16_t* sbase = (const uint16_t*)scales + gidx;
        const uint16_t* bbase = (const uint16_t*)biases + gidx;
        uint32_t qdst[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) qdst[q] = (uint32_t)(jr * ROWB + (((4 * jq + q) ^ nkey(jr)) << 4));

        XChunk<XF> xv[D][8];
        uint32_t cv[D][BITS];
        uint16_t sv[D][2];
        // the stored adapter's slab: thread pt < 128 (waves 4 and 5) copies
        // bytes 16 pt .. +15 of the stage's 2 KB of B
        u32x4_t zv[D];
        const bool zst = FZ && lora.stored && pw < 2;
        const uint16_t* zsrc = (const uint16_t*)lora.a + pt * 8;
        auto issue = [&](int st, int r) {
            const int sc = st < nst ? st : nst - 1;
            const uint8_t* xb = xbase + (int64_t)sc * 64 * XChunk<XF>::EB;
#pragma unroll
            for (int i = 0; i < 8; ++i) xv[r][i].load(xb + xoff[i]);
            if constexpr (FZ) {
                if (zst) zv[r] = *(gv_t)(zsrc + (int64_t)sc * 64 * 16);
            }
            const int64_t row = (int64_t)sc * 64 + jr;
            const uint32_t* ws = wbase + row * wpr;
            if constexpr (BITS % 4 == 0) {
#pragma unroll
                for (int q = 0; q < BITS / 4; ++q) {
                    const u32x4_t v = *((gv_t)ws + q);
                    cv[r][4 * q] = v[0]; cv[r][4 * q + 1] = v[1];
                    cv[r][4 * q + 2] = v[2]; cv[r][4 * q + 3] = v[3];
                }
            } else {
#pragma unroll
                for (int q = 0; q < BITS; ++q) cv[r][q] = *((gw_t)ws + q);
            }
            sv[r][0] = *(gh_t)(sbase + row * G);
            sv[r][1] = *(gh_t)(bbase + row * G);
        };
#pragma unroll
        for (int r = 0; r < D; ++r) issue(r, r);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();  // pairs with the MFMA waves' first barrier
        asm volatile("" ::: "memory");
        for (int s0 = 0; s0 < nst; s0 += 2) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int st = s0 + u;
                uint8_t* xs = u ? xs1 : xs0;
                uint8_t* bq = u ? bq1 : bq0;
#pragma unroll
                for (int i = 0; i < 8; ++i) *(u32x4_t*)(xs + xdst[i]) = xv[u][i].bf16();
                uint32_t d[16];
                dequant_run_fast<BITS>(cv[u], dt_traits<SDT>::to_f32(sv[u][0]),
                                       dt_traits<SDT>::to_f32(sv[u][1]), d);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *(u32x4_t*)(bq + qdst[q]) = u32x4_t{d[4 * q], d[4 * q + 1], d[4 * q + 2], d[4 * q + 3]};
                if constexpr (FZ) {
                    if (zst) *(u32x4_t*)(zb[u] + pt * 16) = zv[u];
                }
                issue(st + D, u);
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this stage's LDS writes are done
                asm volatile("" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
            }
        }
        if constexpr (FZ) {
            // the MFMA waves' two barriers of the down-projection exchange
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
        }
        return;
    }

    // -------------------------------------------------------------- consumers
    if (RQ_K64_CPRIO) __builtin_amdgcn_s_setprio(RQ_K64_CPRIO);
    const int wm = wave >> 1, wn = wave & 1;
    const int lg = lane >> 4, lr = lane & 15;
    f32x4_t acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    uint32_t aoff[2][TM];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            const int row = wm * 128 + a * 16 + lr;
            aoff[h][a] = (uint32_t)(row * 128 + (((h * 4 + lg) ^ (row & 7)) * 16));
        }
    // weight fragment (k-step h, column subtile b), half v: rows 32 h + 8 lg +
    // 4 v + lr / 4, columns wn * 64 + 16 b + 4 (lr % 4) .. +3 (the source side
    // of the transposed read); row % 8 does not depend on h or lg
    uint32_t boff[2][TN];
#pragma unroll
    for (int v = 0; v < 2; ++v)
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const int row = 8 * lg + 4 * v + (lr >> 2);
            const int col = wn * WN + 16 * b + 4 * (lr & 3);
            boff[v][b] = (uint32_t)(row * ROWB + (nchunk(col >> 3, row) << 4) + (col & 7) * 2);
        }
    typedef short s16x4_t __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4_t* lds_s16x4_p;
    // fused down-projection (u = dY . B with a = B^T [16, R]): as in qmm_t_k64.
    // With the adapter as stored (lora.stored: B [R, 16]) a lane's fragment
    // (rank lr, weight rows 8 lg .. +7 of its k-step) comes from the stage's
    // LDS slab of B with two transposed reads, like the weight fragments:
    // source lane 4 s + c of a 16-lane group reads ranks 4 c .. +3 of row s.
    f32x4_t accz[TM];
    u32x4_t zfa_cur = {0u, 0u, 0u, 0u}, zfa_nxt = zfa_cur;
    const uint16_t* zarow = nullptr;
    uint32_t zoff[2] = {0u, 0u};
    // wn as a wave-uniform (scalar) value selects the main loop's
    // instantiation (an EXEC-masked MFMA would still run)
    const int wn_s = __builtin_amdgcn_readfirstlane(wn);
    if constexpr (FZ) {
#pragma unroll
        for (int a = 0; a < TM; ++a) accz[a] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        if (lora.stored) {
#pragma unroll
            for (int v = 0; v < 2; ++v)
                zoff[v] = (uint32_t)((32 * wn + 8 * lg + 4 * v + (lr >> 2)) * 32 + (lr & 3) * 8);
        } else {
            zarow = (const uint16_t*)lora.a + (int64_t)lr * lora.a_ld + 32 * wn + 8 * lg;
            zfa_nxt = *(const u32x4_t*)zarow;
        }
    }

    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // the producers' initial barrier
    asm volatile("" ::: "memory");
    // one instantiation per value of wn in the fused form, as in qmm_t_k64
    auto main_loop = [&](auto zh_c) {
        constexpr int ZH = decltype(zh_c)::value;
        for (int s0 = 0; s0 < nst; s0 += 2) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int st = s0 + u;
                __builtin_amdgcn_s_waitcnt(0xc07f);  // own LDS reads of the previous stage are done
                asm volatile("" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                if (st < nst) {
                    const uint8_t* xs = u ? xs1 : xs0;
                    uint8_t* bq = u ? bq1 : bq0;
                    if constexpr (FZ) {
                        if (lora.stored) {
                            const s16x4_t lo =
                                __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_p)(zb[u] + zoff[0]));
                            const s16x4_t hi =
                                __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_p)(zb[u] + zoff[1]));
                            typedef short s16x8_t __attribute__((ext_vector_type(8)));
                            const s16x8_t v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                            zfa_cur = __builtin_bit_cast(u32x4_t, v);
                        } else {
                            zfa_cur = zfa_nxt;
                            if (st + 1 < nst) zfa_nxt = *(const u32x4_t*)(zarow + (int64_t)(st + 1) * 64);
                        }
                    }
                    // fragments software-pipelined as in qmm_t_k64
                    bf16x8_t bf[2][TN], af[3];
                    auto rdA = [&](int h, int a) {
                        return __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(xs + aoff[h][a]));
                    };
                    auto rdB = [&](int h, int b) {
                        const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (lds_s16x4_p)(bq + boff[0][b] + h * 32 * ROWB));
                        const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (lds_s16x4_p)(bq + boff[1][b] + h * 32 * ROWB));
                        typedef short s16x8_t __attribute__((ext_vector_type(8)));
                        const s16x8_t v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        return __builtin_bit_cast(bf16x8_t, v);
                    };
#pragma unroll
                    for (int b = 0; b < TN; ++b) bf[0][b] = rdB(0, b);
                    af[0] = rdA(0, 0);
                    af[1] = rdA(0, 1);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
#pragma unroll
                        for (int a = 0; a < TM; ++a) {
                            const int q = h * TM + a + 2;
                            if (q < 2 * TM) af[q % 3] = rdA(q / TM, q % TM);
                            if (h == 0 && a == (TM > 2 ? 2 : TM - 1)) {
#pragma unroll
                                for (int b = 0; b < TN; ++b) bf[1][b] = rdB(1, b);
                            }
                            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                            for (int b = 0; b < TN; ++b)
                                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                    bf[h][b], af[(h * TM + a) % 3], acc[a][b], 0, 0, 0);
                            if constexpr (FZ) {
                                if (h == ZH)  // folds: h and ZH are both constants here
                                    accz[a] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                        __builtin_bit_cast(bf16x8_t, zfa_cur), af[(h * TM + a) % 3],
                                        accz[a], 0, 0, 0);
                            }
                            __builtin_amdgcn_sched_barrier(0);
                        }
                    }
                }
            }
        }
    };
    if (FZ && wn_s != 0)
        main_loop(std::integral_constant<int, 1>{});
    else
        main_loop(std::integral_constant<int, 0>{});

    // after the last barrier the ring slot of stage nst - 2 (nst & 1) is free
    if constexpr (FZ) {
        __builtin_amdgcn_s_waitcnt(0xc07f);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();  // every wave is done with both ring slots
        asm volatile("" ::: "memory");
        fused_lora_tail<TM, TN>(acc, accz, (float*)((nst & 1) ? xs0 : xs1), wm, wn, lane, lora,
                                lora.z_out != nullptr && k0 == 0 && wn == 0, M, K, m0 + wm * 128,
                                k0 + wn * WN);
    } else if (lora.z) {
        lora_epilogue<TM, TN>(acc, lora, M, K, m0 + wm * 128, k0 + wn * WN, lane);
    }
    store_wave_tile<TM, TN>(acc, ((nst & 1) ? xs1 : xs0) + wave * 8192, y, y_dt, M, K,
                            m0 + wm * 128, k0 + wn * WN, lane);
}

}  // namespace

namespace rq {

#define RQ_CAT2(a, b) a##b
#define RQ_CAT(a, b) RQ_CAT2(a, b)

hipError_t RQ_CAT(launch_qmm_t_b, RQ_BITS)(const void* x, int x_dt, const uint32_t* wq,
                                      const void* scales, const void* biases, int sb_dt,
                                      int64_t m, int64_t rows, int64_t cols, int gs, void* y,
                                      int y_dt, hipStream_t stream, const LoraArgs* lora) {
    const int gs_shift = __builtin_ctz(gs);
    const LoraArgs lo = lora ? *lora : LoraArgs{nullptr, nullptr, 0, 0.f};
    // bf16 or fp32 activations (fp32 rounded to bf16 as the producers stage them)
    const bool k64 = m >= 256 && (x_dt == RQ_BF16 || x_dt == RQ_F32) && RQ_GEMM_K64 &&
                     sb_dt != RQ_F32 && cols % 64 == 0 && (cols / gs) % 8 == 0 &&
                     (((uintptr_t)x | (uintptr_t)scales | (uintptr_t)biases) & 15) == 0;
    const bool xf = x_dt == RQ_F32;
    if (lora && lora->a) {
        // the fused QLoRA layer with its down-projection in the kernel: rank 16,
        // 4- or 8-bit codes, 128-column tiles (the 160-column ones have no
        // registers left for the extra accumulators)
#if RQ_BITS == 4 || RQ_BITS == 8
        if (!k64 || lora->rank != 16) return hipErrorNotSupported;
        const int tn = (int)((rows + 127) / 128);
        const int bm = ((m + 255) / 256) * tn < RQ_K64_BM128_BELOW ? 128 : 256;
        const int tm = (int)((m + bm - 1) / bm);
        const int blocks = ((tm * tn + 7) / 8) * 8;
#define RQ_FZ_BMX(SD, GSHV, BMV, XFV)                                                             \
    hipLaunchKernelGGL((qmm_t_k64<RQ_BITS, SD, 128, GSHV, BMV, true, XFV>), dim3(blocks),         \
                       dim3(kWsBlock), 0, stream, x, wq, scales, biases, m, rows, cols, y, y_dt,   \
                       tm, tn, lo, 1, nullptr)
#define RQ_FZ_BM(SD, GSHV, BMV) \
    if (xf) { RQ_FZ_BMX(SD, GSHV, BMV, true); } else { RQ_FZ_BMX(SD, GSHV, BMV, false); }
#define RQ_FZ(SD, GSHV) \
    if (bm == 256) { RQ_FZ_BM(SD, GSHV, 256); } else { RQ_FZ_BM(SD, GSHV, 128); }
#define RQ_FZ_GS(SD)                          \
    switch (gs_shift) {                       \
        case 5: RQ_FZ(SD, 5); break;          \
        case 6: RQ_FZ(SD, 6); break;          \
        default: RQ_FZ(SD, 7); break;         \
    }
        if (sb_dt == RQ_BF16) { RQ_FZ_GS(RQ_BF16) } else { RQ_FZ_GS(RQ_F16) }
#undef RQ_FZ_GS
#undef RQ_FZ
#undef RQ_FZ_BM
#undef RQ_FZ_BMX
        return hipGetLastError();
#else
        return hipErrorNotSupported;
#endif
    }
    // 64-wide stages: 16-bit 16-byte aligned scales, whole 8-group chunks
    if (k64) {
        // 160-row tiles (whole rounds over 256 CUs for the 2560-wide RWKV-7 shapes) split
        // evenly into 8-code dequant jobs only at 4 bits
        int bn = (RQ_BITS == 4 && rows % 160 == 0) ? 160 : 128;
        int tn = (int)((rows + bn - 1) / bn);
        // 128-row tiles when 256-row ones leave most CUs idle (small M, narrow R)
        int bm = ((m + 255) / 256) * tn < RQ_K64_BM128_BELOW ? 128 : 256;
        // and at 4 bits 64 x 96 tiles when 128-row ones still leave half of them idle
        // (M = 512 with 2560 outputs: 216 tiles instead of 64)
        if (RQ_BITS == 4 && bm == 128 && ((m + 127) / 128) * tn < RQ_K64_BM64_BELOW) {
            bm = 64;
            bn = 96;
            tn = (int)((rows + bn - 1) / bn);
        }
        const int tm = (int)((m + bm - 1) / bm);
        const int blocks = ((tm * tn + 7) / 8) * 8;
#define RQ_K64_BMX(SD, BNV, GSHV, BMV, XFV)                                                       \
    hipLaunchKernelGGL((qmm_t_k64<RQ_BITS, SD, BNV, GSHV, BMV, false, XFV>), dim3(blocks),        \
                       dim3(kWsBlock), 0, stream, x, wq, scales, biases, m, rows, cols, y, y_dt,   \
                       tm, tn, lo, 1, nullptr)
#define RQ_K64_BM(SD, BNV, GSHV, BMV) \
    if (xf) { RQ_K64_BMX(SD, BNV, GSHV, BMV, true); } else { RQ_K64_BMX(SD, BNV, GSHV, BMV, false); }
#define RQ_K64(SD, BNV, GSHV)                                                                     \
    if (bm == 256) { RQ_K64_BM(SD, BNV, GSHV, 256); } else { RQ_K64_BM(SD, BNV, GSHV, 128); }
#define RQ_K64_GS(SD, BNV)                                                                        \
    switch (gs_shift) {                                                                           \
        case 5: RQ_K64(SD, BNV, 5); break;                                                        \
        case 6: RQ_K64(SD, BNV, 6); break;                                                        \
        default: RQ_K64(SD, BNV, 7); break;                                                       \
    }
#if RQ_BITS == 4
#define RQ_K64_SMALL(SD)                                                                          \
    switch (gs_shift) {                                                                           \
        case 5: RQ_K64_BM(SD, 96, 5, 64); break;                                                  \
        case 6: RQ_K64_BM(SD, 96, 6, 64); break;                                                  \
        default: RQ_K64_BM(SD, 96, 7, 64); break;                                                 \
    }
        if (bm == 64) {
            if (sb_dt == RQ_BF16) { RQ_K64_SMALL(RQ_BF16) } else { RQ_K64_SMALL(RQ_F16) }
        } else if (sb_dt == RQ_BF16) {
            if (bn == 160) { RQ_K64_GS(RQ_BF16, 160) } else { RQ_K64_GS(RQ_BF16, 128) }
        } else {
            if (bn == 160) { RQ_K64_GS(RQ_F16, 160) } else { RQ_K64_GS(RQ_F16, 128) }
        }
#undef RQ_K64_SMALL
#else
        if (sb_dt == RQ_BF16) { RQ_K64_GS(RQ_BF16, 128) } else { RQ_K64_GS(RQ_F16, 128) }
#endif
#undef RQ_K64_GS
#undef RQ_K64
#undef RQ_K64_BM
#undef RQ_K64_BMX
        return hipGetLastError();
    }
    if (lora) return hipErrorNotSupported;  // the low-rank term rides on the k64 kernels only
    if (m >= 256 && x_dt == RQ_BF16) {
        const int bn = rows % 160 == 0 ? 160 : 128;
        const int tm = (int)((m + 255) / 256);
        const int tn = (int)((rows + bn - 1) / bn);
        const int blocks = ((tm * tn + 7) / 8) * 8;
        // parked scales: 16-bit, 16-byte aligned, whole periods of 8 groups
        const bool sbp = sb_dt != RQ_F32 && (cols / gs) % 8 == 0 &&
                         (((uintptr_t)scales | (uintptr_t)biases) & 15) == 0;
#define RQ_DMA(BNV, SBPV)                                                                        \
    RQ_DISPATCH_DT(sb_dt, SD,                                                                    \
        hipLaunchKernelGGL((qmm_t_ws<RQ_BITS, SD, BNV,                                          \
                                     ws_slots<RQ_BITS, SD, BNV, SBPV && SD != RQ_F32>(),          \
                                     SBPV && SD != RQ_F32>),                                      \
                           dim3(blocks), dim3(kWsBlock), 0, stream, (const uint16_t*)x, wq,      \
                           scales, biases, m,                                                    \
                           rows, cols, gs_shift, y, y_dt, tm, tn))
        if (sbp) {
            if (bn == 160) { RQ_DMA(160, true); } else { RQ_DMA(128, true); }
        } else {
            if (bn == 160) { RQ_DMA(160, false); } else { RQ_DMA(128, false); }
        }
#undef RQ_DMA
        return hipGetLastError();
    }
    if (m >= 256) {
        // weight-row tile: whole rounds over 256 CUs at M=4096 for the RWKV-7 shapes
        const int bn = rows % 160 == 0 ? 160 : 128;
        const int tm = (int)((m + 255) / 256);
        const int tn = (int)((rows + bn - 1) / bn);
        const int blocks = ((tm * tn + 7) / 8) * 8;
#define RQ_BIG(BNV)                                                                          \
    RQ_DISPATCH_DT(x_dt, XD,                                                                 \
        hipLaunchKernelGGL((qmm_t_big<RQ_BITS, XD, BNV>), dim3(blocks), dim3(kBlock), 0, stream, \
                           x, wq, scales, biases, sb_dt, m, rows, cols, gs_shift, y, y_dt, tm, tn))
        if (bn == 160) { RQ_BIG(160); } else { RQ_BIG(128); }
#undef RQ_BIG
        return hipGetLastError();
    }
    constexpr int BM = 128;
    const dim3 grid((unsigned)((rows + BN - 1) / BN), (unsigned)((m + BM - 1) / BM));
    RQ_DISPATCH_DT(x_dt, XD,
        hipLaunchKernelGGL((qmm_t_kernel<RQ_BITS, XD, BM>), grid, dim3(kBlock), 0, stream, x, wq,
                           scales, biases, sb_dt, m, rows, cols, gs_shift, y, y_dt));
    return hipGetLastError();
}

// Split-K form of the 64-wide-stage GEMM (transpose=1; the caller checked the
// k64 conditions): `splits` blocks per bm x bn output tile, each over a whole
// number of 8-group periods of the contraction, fp32 partial tiles into
// part[splits][m][rows] (launch_splitk_reduce sums them in split order).
hipError_t RQ_CAT(launch_qmm_t_splitk_b, RQ_BITS)(const void* x, int x_dt, const uint32_t* wq,
                                             const void* scales, const void* biases, int sb_dt,
                                             int64_t m, int64_t rows, int64_t cols, int gs,
                                             int bm, int splits, float* part, hipStream_t stream) {
    const int gs_shift = __builtin_ctz(gs);
    const int bn = (RQ_BITS == 4 && rows % 160 == 0) ? 160 : 128;
    const int tn = (int)((rows + bn - 1) / bn), tm = (int)((m + bm - 1) / bm);
    const int blocks = ((tm * tn * splits + 7) / 8) * 8;
    const bool xf = x_dt == RQ_F32;
    const LoraArgs lo{nullptr, nullptr, 0, 0.f};
#define RQ_SK(SD, BNV, GSHV, BMV, XFV)                                                            \
    hipLaunchKernelGGL((qmm_t_k64<RQ_BITS, SD, BNV, GSHV, BMV, false, XFV>), dim3(blocks),        \
                       dim3(kWsBlock), 0, stream, x, wq, scales, biases, m, rows, cols, nullptr,  \
                       (int)RQ_F32, tm, tn, lo, splits, part)
#define RQ_SK_X(SD, BNV, GSHV, BMV) \
    if (xf) { RQ_SK(SD, BNV, GSHV, BMV, true); } else { RQ_SK(SD, BNV, GSHV, BMV, false); }
#define RQ_SK_BM(SD, BNV, GSHV) \
    if (bm == 256) { RQ_SK_X(SD, BNV, GSHV, 256); } else { RQ_SK_X(SD, BNV, GSHV, 128); }
#define RQ_SK_GS(SD, BNV)                  \
    switch (gs_shift) {                    \
        case 5: RQ_SK_BM(SD, BNV, 5); break; \
        case 6: RQ_SK_BM(SD, BNV, 6); break; \
        default: RQ_SK_BM(SD, BNV, 7); break; \
    }
#if RQ_BITS == 4
    if (bn == 160) {
        if (sb_dt == RQ_BF16) { RQ_SK_GS(RQ_BF16, 160) } else { RQ_SK_GS(RQ_F16, 160) }
        return hipGetLastError();
    }
#endif
    if (sb_dt == RQ_BF16) { RQ_SK_GS(RQ_BF16, 128) } else { RQ_SK_GS(RQ_F16, 128) }
#undef RQ_SK_GS
#undef RQ_SK_BM
#undef RQ_SK_X
#undef RQ_SK
    return hipGetLastError();
}

hipError_t RQ_CAT(launch_qmm_n_b, RQ_BITS)(const void* x, int x_dt, const uint32_t* wq,
                                      const void* scales, const void* biases, int sb_dt,
                                      int64_t m, int64_t rows, int64_t cols, int gs, void* y,
                                      int y_dt, hipStream_t stream, const LoraArgs* lora) {
    const LoraArgs lo = lora ? *lora : LoraArgs{nullptr, nullptr, 0, 0.f};
    // warp-specialised transposed GEMM: bf16 dY, 16-bit aligned scales,
    // whole stages of 64 weight rows and whole tiles of 128 or 160 output
    // columns (160: 4- and 8-bit codes)
    const bool can128 = cols % 128 == 0;
    const bool can160 = (RQ_BITS == 4 || RQ_BITS == 8) && RQ_GEMM_N160 && cols % 160 == 0;
    // bf16 or fp32 dY (fp32 rounded to bf16 as the producers stage it)
    const bool k64 = m >= 256 && (x_dt == RQ_BF16 || x_dt == RQ_F32) && RQ_GEMM_K64 &&
                     sb_dt != RQ_F32 && rows % 64 == 0 && (can128 || can160) &&
                     ((uintptr_t)x & 15) == 0 && (((uintptr_t)scales | (uintptr_t)biases) & 7) == 0;
    const bool xf = x_dt == RQ_F32;
#define RQ_NK64(SD, BNV, FZV)                                                                       \
    do {                                                                                           \
        if (xf)                                                                                    \
            hipLaunchKernelGGL((qmm_n_k64<RQ_BITS, SD, BNV, FZV, true>), dim3(blocks),            \
                               dim3(kWsBlock), 0, stream, x, wq, scales, biases, m, rows, cols,   \
                               __builtin_ctz(gs), y, y_dt, tm, tn, lo);                           \
        else                                                                                       \
            hipLaunchKernelGGL((qmm_n_k64<RQ_BITS, SD, BNV, FZV, false>), dim3(blocks),           \
                               dim3(kWsBlock), 0, stream, x, wq, scales, biases, m, rows, cols,   \
                               __builtin_ctz(gs), y, y_dt, tm, tn, lo);                           \
    } while (0)
    if (lora && lora->a) {
        // the fused QLoRA layer's dX with u = dY . B in the kernel (rank 16,
        // 4- or 8-bit codes)
#if RQ_BITS == 4 || RQ_BITS == 8
        if (!k64 || !can128 || lora->rank != 16) return hipErrorNotSupported;
        const int tm = (int)((m + 255) / 256);
        const int tn = (int)(cols / 128);
        const int blocks = ((tm * tn + 7) / 8) * 8;
        if (sb_dt == RQ_BF16) RQ_NK64(RQ_BF16, 128, true);
        else RQ_NK64(RQ_F16, 128, true);
        return hipGetLastError();
#else
        return hipErrorNotSupported;
#endif
    }
    if (k64) {
        const int tm = (int)((m + 255) / 256);
        // 160-column tiles where 128-column ones do not divide the output or
        // take more rounds of 256 CUs than it costs to run fewer, wider tiles:
        // a 160-column tile runs ~1.35x as long as a 128-column one (65.8 vs
        // 48.6 us per round at R = 2560, M = 4096), so 2560-wide outputs (one
        // round of 256 instead of two of 320) and 10240-wide ones at M = 2048
        // (2 rounds of 512 against 3 of 640) take them, 10240-wide ones at
        // M = 4096 (4 rounds of 1024 against 5 of 1280) do not
        auto rounds = [&](int64_t nt) { return (double)((nt + kK64Cus - 1) / kK64Cus); };
        const bool wide = can160 && (!can128 || 1.35 * rounds((int64_t)tm * (cols / 160)) <
                                                    rounds((int64_t)tm * (cols / 128)));
        const int tn = (int)(cols / (wide ? 160 : 128));
        const int blocks = ((tm * tn + 7) / 8) * 8;
#if RQ_BITS == 4 || RQ_BITS == 8
        if (wide) {
            if (sb_dt == RQ_BF16) RQ_NK64(RQ_BF16, 160, false);
            else RQ_NK64(RQ_F16, 160, false);
            return hipGetLastError();
        }
#endif
        if (sb_dt == RQ_BF16) RQ_NK64(RQ_BF16, 128, false);
        else RQ_NK64(RQ_F16, 128, false);
        return hipGetLastError();
    }
#undef RQ_NK64
    if (lora) return hipErrorNotSupported;  // the low-rank term rides on the k64 kernels only
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
