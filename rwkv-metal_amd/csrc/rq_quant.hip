// rq_quant.hip -- quantize / dequantize / pack / unpack kernels (gfx950).
//
// All four are HBM-bound streaming kernels.  One thread owns one run of 32
// consecutive codes of a row (BITS whole packed words), so every thread reads
// and writes whole, aligned words and no two threads share an output word.
// Consecutive threads own consecutive runs, so a wave's 64 runs are one
// contiguous range of the dense side; dequantize stores that range 1 KB per
// instruction after moving it through LDS.
#include "rq_common.h"
#include "rq_launch.h"

namespace {

constexpr int kBlock = 256;

// --------------------------------------------------------------- quantize
//
// Affine quantize of MLX (mx.quantize), reached from nn.quantize at
// rwkv_metal/lora/finetune.py:88-89.  A group of gs values spans gs/32
// consecutive threads; min and max are combined with xor-shuffles inside that
// lane group.  The scale/bias arithmetic is single precision with IEEE
// division (hipcc's default for '/') and rintf (round half to even), in the
// same order as MLX's CPU quantizer.
template <int BITS, int WDT>
__global__ __launch_bounds__(kBlock) void quantize_kernel(
    const void* __restrict__ w, int64_t rows, int64_t cols, int gs_shift,
    uint32_t* __restrict__ wq, void* __restrict__ scales, void* __restrict__ biases) {
    const int64_t runs_per_row = cols >> 5;
    const int64_t total = rows * runs_per_row;
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int lpg = 1 << (gs_shift - 5);  // lanes per group: 1, 2 or 4
    // Threads past the end still take part in the shuffles (their lane group
    // is entirely past the end because total is a multiple of lpg).
    const bool live = t < total;
    const int64_t tt = live ? t : 0;
    const int64_t row = tt / runs_per_row;
    const int64_t run = tt - row * runs_per_row;

    // (Loading the wave's 2048 inputs 1 KB per instruction through LDS, the
    // way dequantize stores, measured slower here: 3.2 vs 3.8 TB/s at 4 bits.)
    float v[32];
    load32_f32<WDT>(w, row * cols + run * 32, v);

    float w_min = v[0], w_max = v[0];
#pragma unroll
    for (int j = 1; j < 32; ++j) {
        w_min = fminf(w_min, v[j]);
        w_max = fmaxf(w_max, v[j]);
    }
    for (int o = 1; o < lpg; o <<= 1) {
        w_min = fminf(w_min, __shfl_xor(w_min, o, 64));
        w_max = fmaxf(w_max, __shfl_xor(w_max, o, 64));
    }

    const float n_bins = (float)((1 << BITS) - 1);
    const float eps = 1e-7f;
    const bool side = fabsf(w_min) > fabsf(w_max);
    float scale = fmaxf((w_max - w_min) / n_bins, eps);
    scale = side ? scale : -scale;
    const float edge = side ? w_min : w_max;
    const float q0 = rintf(edge / scale);
    float bias = 0.0f;
    if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
    }

    // code = clip(rint((w - bias) / scale)) with the IEEE quotient.  The
    // quotient only matters through rint, so it is first approximated as
    // (w - bias) * rcp(scale): v_rcp_f32 is within 1 ulp, so for |quotient|
    // <= 512 the product is within 2^-13 of the exact quotient, and where it
    // lies more than 2^-11 away from a half-integer both round to the same
    // integer (ties included: a tie has the product within 2^-13 of .5).
    // Only the rest take the IEEE division.
    const float rs = __builtin_amdgcn_rcpf(scale);
    uint32_t codes[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float d = v[j] - bias;
        float a = d * rs;
        if (!(fabsf(a) <= 512.0f && fabsf(a - floorf(a) - 0.5f) > 0x1p-11f)) a = d / scale;
        float q = rintf(a);
        q = fminf(fmaxf(q, 0.0f), n_bins);
        codes[j] = (uint32_t)q;
    }
    uint32_t words[BITS];
    run_pack<BITS>(codes, words);
    if (!live) return;
    store_run<BITS>(wq + row * (runs_per_row * BITS) + run * BITS, words);
    if ((run & (lpg - 1)) == 0) {
        const int64_t gi = row * (cols >> gs_shift) + (run >> (gs_shift - 5));
        typedef typename dt_traits<WDT>::storage S;
        ((S*)scales)[gi] = dt_traits<WDT>::from_f32(scale);
        ((S*)biases)[gi] = dt_traits<WDT>::from_f32(bias);
    }
}

// ------------------------------------------------------------- dequantize
//
// mx.dequantize: ŵ = T(T(code*scale) + bias), T = the scales dtype (MLX
// evaluates multiply and add as two ops in that dtype).  __fmul_rn/__fadd_rn
// keep the two roundings separate when T is f32.
template <int BITS, int ODT>
// One thread per 32-code run.  With idx != NULL this is the embedding
// lookup: output row r is table row idx[r] (rows = number of indices,
// src_rows = table rows); an index outside the table gives a row of NaN and
// reads nothing.
__global__ __launch_bounds__(kBlock) void dequantize_kernel(
    const uint32_t* __restrict__ wq, const void* __restrict__ scales,
    const void* __restrict__ biases, int sb_dt, int64_t rows, int64_t cols, int gs_shift,
    void* __restrict__ out, const int64_t* __restrict__ idx, int64_t src_rows) {
    // A lane's 32 outputs (64 or 128 B) are staged through LDS so that each
    // store instruction of the wave writes 1 KB contiguous: the wave's 64
    // runs are 2048 consecutive outputs (run t lands at t * 32).  Stored
    // straight from registers, the four 16-B stores of a lane sat 64 B apart,
    // one request per lane and instruction.  Lane L's chunk i sits at LDS
    // chunk L*(NC+1) + i (the pad spreads the banks).
    constexpr int NC = ODT == RQ_F32 ? 8 : 4;  // 16-byte chunks per lane
    __shared__ __attribute__((aligned(16))) uint4 stg[kBlock / 64][64 * (NC + 1)];
    const int64_t runs_per_row = cols >> 5;
    const int64_t total = rows * runs_per_row;
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int lane = threadIdx.x & 63;
    const bool live = t < total;
    const int64_t tt = live ? t : total - 1;
    const int64_t row = tt / runs_per_row;
    const int64_t run = tt - row * runs_per_row;
    const int64_t src = idx ? idx[row] : row;
    float vals[32];
    if (src < 0 || src >= src_rows) {
#pragma unroll
        for (int j = 0; j < 32; ++j) vals[j] = __builtin_nanf("");
    } else {
        const int64_t gi = src * (cols >> gs_shift) + (run >> (gs_shift - 5));
        const float s = load_dt(scales, sb_dt, gi);
        const float b = load_dt(biases, sb_dt, gi);

        uint32_t words[BITS];
        load_run<BITS>(wq + src * (runs_per_row * BITS) + run * BITS, words);
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const float c = (float)run_code<BITS>(words, j);
            const float p = round_to_dt(sb_dt, __fmul_rn(c, s));
            vals[j] = round_to_dt(sb_dt, __fadd_rn(p, b));
        }
    }
    uint4* line = stg[threadIdx.x >> 6];
    if constexpr (ODT == RQ_F32) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            line[lane * (NC + 1) + i] =
                make_uint4(__float_as_uint(vals[4 * i]), __float_as_uint(vals[4 * i + 1]),
                           __float_as_uint(vals[4 * i + 2]), __float_as_uint(vals[4 * i + 3]));
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t d[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t lo = dt_traits<ODT>::from_f32(vals[8 * i + 2 * j]);
                const uint32_t hi = dt_traits<ODT>::from_f32(vals[8 * i + 2 * j + 1]);
                d[j] = lo | (hi << 16);
            }
            line[lane * (NC + 1) + i] = make_uint4(d[0], d[1], d[2], d[3]);
        }
    }
    __builtin_amdgcn_wave_barrier();  // LDS runs in order within the wave
    const int64_t t0 = t - lane;      // the wave's first run
    uint4* dst = (uint4*)((uint8_t*)out + t0 * (32 * (ODT == RQ_F32 ? 4 : 2)));
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = lane + 64 * i;  // chunk c of the wave's output: lane c / NC, its chunk c % NC
        const uint4 v = line[(c / NC) * (NC + 1) + c % NC];
        if (t0 + c / NC < total) dst[c] = v;
    }
}

// ---------------------------------------------------------- pack / unpack

template <int BITS>
__global__ __launch_bounds__(kBlock) void pack_kernel(const uint8_t* __restrict__ codes,
                                                       int64_t rows, int64_t cols,
                                                       uint32_t* __restrict__ wq) {
    const int64_t runs_per_row = cols >> 5;
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= rows * runs_per_row) return;
    const uint4* src = (const uint4*)(codes + t * 32);  // run t = codes[t*32 .. t*32+31]
    uint32_t c[32];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint4 v = src[i];
        uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                c[16 * i + 4 * j + b] = ((w4[j] >> (8 * b)) & 0xffu) & ((1u << BITS) - 1u);
    }
    uint32_t words[BITS];
    run_pack<BITS>(c, words);
    store_run<BITS>(wq + t * BITS, words);
}

template <int BITS>
__global__ __launch_bounds__(kBlock) void unpack_kernel(const uint32_t* __restrict__ wq,
                                                         int64_t rows, int64_t cols,
                                                         uint8_t* __restrict__ codes) {
    const int64_t runs_per_row = cols >> 5;
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= rows * runs_per_row) return;
    uint32_t words[BITS];
    load_run<BITS>(wq + t * BITS, words);
    uint32_t packed[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        packed[i] = run_code<BITS>(words, 4 * i) | (run_code<BITS>(words, 4 * i + 1) << 8) |
                    (run_code<BITS>(words, 4 * i + 2) << 16) |
                    (run_code<BITS>(words, 4 * i + 3) << 24);
    }
    uint4* dst = (uint4*)(codes + t * 32);
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
}

inline int grid_for(int64_t threads) { return (int)((threads + kBlock - 1) / kBlock); }

}  // namespace

// Split-K reduction: y = sum over splits s = 0, 1, .. of part[s] (fp32 partial
// products of a split GEMM, [splits][n]), added in split order (the same bits
// on every run), rounded once into y's dtype.  Four consecutive outputs per
// thread when vec (rows % 4 == 0), one otherwise.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part,
                                                            int splits, int64_t n,
                                                            void* __restrict__ y, int y_dt,
                                                            bool vec) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (vec) {
        const int64_t i = 4 * t;
        if (i >= n) return;
        f32x4_t acc = *(const f32x4_t*)(part + i);
        for (int s = 1; s < splits; ++s) acc += *(const f32x4_t*)(part + (int64_t)s * n + i);
        if (y_dt == RQ_F32) {
            *(f32x4_t*)((float*)y + i) = acc;
        } else {
            typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
            const u32x2_t v = y_dt == RQ_BF16
                ? u32x2_t{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])}
                : u32x2_t{f32_to_f16_bits(acc[0]) | (f32_to_f16_bits(acc[1]) << 16),
                          f32_to_f16_bits(acc[2]) | (f32_to_f16_bits(acc[3]) << 16)};
            *(u32x2_t*)((uint16_t*)y + i) = v;
        }
        return;
    }
    if (t >= n) return;
    float acc = part[t];
    for (int s = 1; s < splits; ++s) acc += part[(int64_t)s * n + t];
    store_dt(y, y_dt, t, acc);
}

namespace rq {

hipError_t launch_quantize(const void* w, int w_dt, int64_t rows, int64_t cols, int gs,
                           int bits, uint32_t* wq, void* scales, void* biases,
                           hipStream_t stream) {
    const int64_t threads = rows * (cols / 32);
    if (threads == 0) return hipSuccess;
    const int gs_shift = __builtin_ctz(gs);
    RQ_DISPATCH_BITS(bits, B, RQ_DISPATCH_DT(w_dt, D,
        hipLaunchKernelGGL((quantize_kernel<B, D>), dim3(grid_for(threads)), dim3(kBlock), 0,
                           stream, w, rows, cols, gs_shift, wq, scales, biases)));
    return hipGetLastError();
}

hipError_t launch_dequantize(const uint32_t* wq, const void* scales, const void* biases,
                             int sb_dt, int64_t rows, int64_t cols, int gs, int bits, void* out,
                             int out_dt, hipStream_t stream) {
    const int64_t threads = rows * (cols / 32);
    if (threads == 0) return hipSuccess;
    const int gs_shift = __builtin_ctz(gs);
    RQ_DISPATCH_BITS(bits, B, RQ_DISPATCH_DT(out_dt, D,
        hipLaunchKernelGGL((dequantize_kernel<B, D>), dim3(grid_for(threads)), dim3(kBlock), 0,
                           stream, wq, scales, biases, sb_dt, rows, cols, gs_shift, out,
                           (const int64_t*)nullptr, rows)));
    return hipGetLastError();
}

hipError_t launch_embedding(const int64_t* idx, int64_t n, const uint32_t* wq,
                            const void* scales, const void* biases, int sb_dt, int64_t rows,
                            int64_t cols, int gs, int bits, void* out, int out_dt,
                            hipStream_t stream) {
    const int64_t threads = n * (cols / 32);
    if (threads == 0) return hipSuccess;
    const int gs_shift = __builtin_ctz(gs);
    RQ_DISPATCH_BITS(bits, B, RQ_DISPATCH_DT(out_dt, D,
        hipLaunchKernelGGL((dequantize_kernel<B, D>), dim3(grid_for(threads)), dim3(kBlock), 0,
                           stream, wq, scales, biases, sb_dt, n, cols, gs_shift, out, idx,
                           rows)));
    return hipGetLastError();
}

hipError_t launch_pack(const uint8_t* codes, int64_t rows, int64_t cols, int bits, uint32_t* wq,
                       hipStream_t stream) {
    const int64_t threads = rows * (cols / 32);
    if (threads == 0) return hipSuccess;
    RQ_DISPATCH_BITS(bits, B,
        hipLaunchKernelGGL((pack_kernel<B>), dim3(grid_for(threads)), dim3(kBlock), 0, stream,
                           codes, rows, cols, wq));
    return hipGetLastError();
}

hipError_t launch_unpack(const uint32_t* wq, int64_t rows, int64_t cols, int bits,
                         uint8_t* codes, hipStream_t stream) {
    const int64_t threads = rows * (cols / 32);
    if (threads == 0) return hipSuccess;
    RQ_DISPATCH_BITS(bits, B,
        hipLaunchKernelGGL((unpack_kernel<B>), dim3(grid_for(threads)), dim3(kBlock), 0, stream,
                           wq, rows, cols, codes));
    return hipGetLastError();
}

hipError_t launch_splitk_reduce(const float* part, int splits, int64_t m, int64_t rows, void* y,
                                int y_dt, hipStream_t stream) {
    const int64_t n = m * rows;
    if (n == 0) return hipSuccess;
    const bool vec = rows % 4 == 0;
    const int64_t threads = vec ? n / 4 : n;
    const dim3 grid((unsigned)((threads + 255) / 256));
    hipLaunchKernelGGL(splitk_reduce_kernel, grid, dim3(256), 0, stream, part, splits, n, y, y_dt,
                       vec);
    return hipGetLastError();
}

}  // namespace rq
