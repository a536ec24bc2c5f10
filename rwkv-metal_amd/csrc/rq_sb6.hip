// rq_sb6.hip -- rwkv-quant "sb6" (K3-interleaved) tensors on gfx950.
//
// The layout RwkvqLinear holds (rwkv_metal/lora/rwkvq_kernel.py:18-25) and its
// arithmetic (rwkv_metal/lora/rwkvq_linear.py:140-175, rwkvq_kernel.py:86-100).
// Blocks are 32 codes of one row:
//   qblk[row, blk] : 16 bytes, byte j = code j (low nibble) | code j+16 (high
//                    nibble); xbits >= 1: +4 bytes, bit c = bit 4 of code c;
//                    xbits == 2: +4 bytes, bit c = bit 5 of code c
//   qsqm[row, blk] : (qs uint8, qm int8)
//   ddm[row, sblk] : (d, dm) float16, sblk = blk / gw_sb
//   scale = f16(qs * d), min = f16(qm * dm), w = code * scale + min in fp32.
// code * scale is exact in fp32 (at most 6 + 11 significant bits), so the
// result is one rounding of the sum whether or not it is contracted.
//
//  * sb6_dequantize_kernel: dense [rows, cols] fp32 or bf16 (RNE), the fused
//    dequantize of RwkvqLinear._dequant_w.
//  * sb6_to_affine_kernel: the one-time repack of RwkvqNativeLinear
//    (rwkv_metal/lora/rwkvq_native.py:49-78, 103-113): codes into the MLX
//    bitstream at bits = 4 + xbits, scale max(scale, 1e-8) and bias = min,
//    fp32, group size 32; w_q may be NULL (RwkvqHybridLinear expands only the
//    scales and biases per forward, rwkvq_hybrid.py:72-86).
// One thread per block; HBM-bound.
#include "rq_common.h"
#include "rq_launch.h"

namespace {

constexpr int kBlock = 256;

template <int XB>
RQ_DEV void sb6_decode(const uint8_t* __restrict__ qblk, int64_t blk_index, uint32_t* codes) {
    constexpr int BB = 16 + 4 * XB;  // bytes per block: 16, 20 or 24 (4-byte aligned)
    const uint32_t* q = (const uint32_t*)(qblk + blk_index * BB);
    uint32_t w[4 + XB];
#pragma unroll
    for (int i = 0; i < 4 + XB; ++i) w[i] = q[i];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint32_t byte = (w[j >> 2] >> (8 * (j & 3))) & 0xffu;
        codes[j] = byte & 0xfu;
        codes[j + 16] = byte >> 4;
    }
#pragma unroll
    for (int x = 0; x < XB; ++x)
#pragma unroll
        for (int c = 0; c < 32; ++c) codes[c] |= ((w[4 + x] >> c) & 1u) << (4 + x);
}

RQ_DEV void sb6_scale_min(const uint8_t* __restrict__ qsqm, const uint16_t* __restrict__ ddm,
                          int64_t blk_index, int64_t dd_index, float& sc, float& mn) {
    const uint32_t sm = *(const uint16_t*)(qsqm + blk_index * 2);
    const uint32_t dd = *(const uint32_t*)(ddm + dd_index * 2);
    const float qs = (float)(sm & 0xffu);
    const float qm = (float)(int8_t)(uint8_t)(sm >> 8);
    // The products are kept as fp32 multiplies: fused with the f16 rounding
    // the compiler forms v_fma_mixlo_f16(a, b, +0), which turns a -0.0
    // product (qm = 0, dm < 0) into +0.0.
    float ps = qs * f16_bits_to_f32(dd & 0xffffu);
    float pm = qm * f16_bits_to_f32(dd >> 16);
    asm("" : "+v"(ps));
    asm("" : "+v"(pm));
    sc = f16_bits_to_f32(f32_to_f16_bits(ps));
    mn = f16_bits_to_f32(f32_to_f16_bits(pm));
}

template <int XB, int ODT>
__global__ __launch_bounds__(kBlock) void sb6_dequantize_kernel(
    const uint8_t* __restrict__ qblk, const uint8_t* __restrict__ qsqm,
    const uint16_t* __restrict__ ddm, int64_t rows, int64_t nb, int gw_sb, void* __restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= rows * nb) return;
    const int64_t row = t / nb, blk = t - row * nb;
    uint32_t codes[32];
    sb6_decode<XB>(qblk, t, codes);
    float sc, mn;
    sb6_scale_min(qsqm, ddm, t, row * (nb / gw_sb) + blk / gw_sb, sc, mn);
    float v[32];
#pragma unroll
    for (int c = 0; c < 32; ++c) v[c] = __fadd_rn(__fmul_rn((float)codes[c], sc), mn);
    const int64_t o = row * nb * 32 + blk * 32;
    if constexpr (ODT == RQ_F32) {
        f32x4_t* dst = (f32x4_t*)((float*)out + o);
#pragma unroll
        for (int i = 0; i < 8; ++i) dst[i] = f32x4_t{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
    } else {
        typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
        u32x4_t* dst = (u32x4_t*)((uint16_t*)out + o);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t d[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                d[j] = dt_traits<ODT>::from_f32(v[8 * i + 2 * j]) |
                       ((uint32_t)dt_traits<ODT>::from_f32(v[8 * i + 2 * j + 1]) << 16);
            dst[i] = u32x4_t{d[0], d[1], d[2], d[3]};
        }
    }
}

template <int XB>
__global__ __launch_bounds__(kBlock) void sb6_to_affine_kernel(
    const uint8_t* __restrict__ qblk, const uint8_t* __restrict__ qsqm,
    const uint16_t* __restrict__ ddm, int64_t rows, int64_t nb, int gw_sb,
    uint32_t* __restrict__ wq, float* __restrict__ scales, float* __restrict__ biases) {
    constexpr int BITS = 4 + XB;
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= rows * nb) return;
    const int64_t row = t / nb, blk = t - row * nb;
    if (wq) {
        uint32_t codes[32], words[BITS];
        sb6_decode<XB>(qblk, t, codes);
        run_pack<BITS>(codes, words);
#pragma unroll
        for (int w = 0; w < BITS; ++w) wq[t * BITS + w] = words[w];  // run t of row-major w_q
    }
    float sc, mn;
    sb6_scale_min(qsqm, ddm, t, row * (nb / gw_sb) + blk / gw_sb, sc, mn);
    scales[t] = sc >= 1e-8f ? sc : 1e-8f;  // mx.maximum(scale, 1e-8)
    biases[t] = mn;
}

inline unsigned grid_for(int64_t threads) { return (unsigned)((threads + kBlock - 1) / kBlock); }

}  // namespace

namespace rq {

hipError_t launch_sb6_dequantize(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                                 int64_t rows, int64_t cols, int gw_sb, int xbits, void* out,
                                 int out_dt, hipStream_t stream) {
    const int64_t nb = cols / 32;
    if (rows * nb == 0) return hipSuccess;
#define RQ_SB6_DQ(XBV)                                                                           \
    RQ_DISPATCH_DT(out_dt, D,                                                                    \
        hipLaunchKernelGGL((sb6_dequantize_kernel<XBV, D>), dim3(grid_for(rows * nb)),           \
                           dim3(kBlock), 0, stream, qblk, qsqm, ddm, rows, nb, gw_sb, out))
    switch (xbits) {
        case 0: RQ_SB6_DQ(0); break;
        case 1: RQ_SB6_DQ(1); break;
        default: RQ_SB6_DQ(2); break;
    }
#undef RQ_SB6_DQ
    return hipGetLastError();
}

hipError_t launch_sb6_to_affine(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                                int64_t rows, int64_t cols, int gw_sb, int xbits, uint32_t* wq,
                                float* scales, float* biases, hipStream_t stream) {
    const int64_t nb = cols / 32;
    if (rows * nb == 0) return hipSuccess;
#define RQ_SB6_AF(XBV)                                                                           \
    hipLaunchKernelGGL((sb6_to_affine_kernel<XBV>), dim3(grid_for(rows * nb)), dim3(kBlock), 0, \
                       stream, qblk, qsqm, ddm, rows, nb, gw_sb, wq, scales, biases)
    switch (xbits) {
        case 0: RQ_SB6_AF(0); break;
        case 1: RQ_SB6_AF(1); break;
        default: RQ_SB6_AF(2); break;
    }
#undef RQ_SB6_AF
    return hipGetLastError();
}

}  // namespace rq
