// rq_lora.hip -- the QLoRA layer's low-rank down-projection (gfx950).
//
//   z[m, j] = sum_k x[m, k] * a[j, k]        (bf16 in and out, fp32 accumulation)
//
// LoRALinear.__call__ (rwkv_metal/lora/lora.py:58-63) computes z = x . A^T in
// the forward, and MLX autograd u = dY . B in the backward (a = B^T there).
// Both are tall and skinny: M x K activations against rank <= 64 rows, so
// the product is bound by reading x once.
//
//  * One block per 16 rows of x, W waves (16 at rank 16, else 8) splitting
//    K by 32-column k-steps (wave w takes k-steps w, w+W, ...).  v_mfma_f32_16x16x32_bf16 with
//    A = x (lane L: row L%16, columns 8(L/16)..+7 of the k-step: one 16-byte
//    load) and B = a^T (lane L: row j0 + L%16 of a, the same columns), one
//    MFMA per 16 ranks.
//  * A wave issues the loads of U k-steps at once (4, 2 at rank > 32) and
//    the next U before the MFMAs of the current ones (two register sets).
//  * The W waves' partial 16 x rank tiles are summed through LDS behind one
//    barrier and stored as bf16.
#include "rq_common.h"
#include "rq_launch.h"

namespace {

// waves per block and k-steps per batch of loads, by rank tiles: two
// register sets of U x (1 + RT) 16-byte loads stay within the VGPRs the
// block size allows (128 at 16 waves, 256 at 8)
template <int RT> struct LoraShape {
    static constexpr int W = RT == 1 ? 16 : 8;
    static constexpr int U = RT <= 2 ? 4 : 2;
};

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int RT>  // rank tiles of 16
__global__ __launch_bounds__(64 * LoraShape<RT>::W) void lora_down_kernel(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, const uint16_t* __restrict__ a,
    uint16_t* __restrict__ z) {
    constexpr int kLoraWaves = LoraShape<RT>::W, U = LoraShape<RT>::U;
    __shared__ __attribute__((aligned(16))) float red[kLoraWaves][RT][4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lg = lane >> 4, lr = lane & 15;
    const int64_t m0 = (int64_t)blockIdx.x * 16;
    const int64_t row = (m0 + lr) < M ? (m0 + lr) : M - 1;  // rows past M: any valid row
    const int nsteps = (int)(K >> 5);
    const uint16_t* xr = x + row * K + lg * 8;
    const uint16_t* ar = a + (int64_t)lr * K + lg * 8;

    f32x4_t acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // Batches of U k-steps, software-pipelined: the loads of batch j + 1 are
    // issued before the MFMAs of batch j.  Loads past the end read the last
    // k-step (valid memory) and are not used.
    u32x4_t xa[2][U], wb[2][U][RT];
    auto load = [&](int b, int s0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int s = s0 + kLoraWaves * u;
            s = s < nsteps ? s : nsteps - 1;
            xa[b][u] = *(const u32x4_t*)(xr + (int64_t)s * 32);
#pragma unroll
            for (int t = 0; t < RT; ++t)
                wb[b][u][t] = *(const u32x4_t*)(ar + ((int64_t)t * 16 * K + (int64_t)s * 32));
        }
    };
    auto mma = [&](int b, int s0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (s0 + kLoraWaves * u < nsteps) {
                const bf16x8_t av = __builtin_bit_cast(bf16x8_t, xa[b][u]);
#pragma unroll
                for (int t = 0; t < RT; ++t)
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        av, __builtin_bit_cast(bf16x8_t, wb[b][u][t]), acc[t], 0, 0, 0);
            }
        }
    };
    constexpr int STEP = kLoraWaves * U;
    load(0, wave);
    int s0 = wave;
    for (; s0 + STEP < nsteps; s0 += 2 * STEP) {
        load(1, s0 + STEP);
        mma(0, s0);
        if (s0 + 2 * STEP >= nsteps) { mma(1, s0 + STEP); s0 += 2 * STEP; break; }
        load(0, s0 + 2 * STEP);
        mma(1, s0 + STEP);
    }
    if (s0 < nsteps) mma(0, s0);
    // lane (lg, lr) holds D[4 lg + i][lr]: rows m0 + 4 lg + i, rank j0 + lr
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][t][i][lane] = acc[t][i];
    __syncthreads();
    if (wave < RT) {
        const int t = wave;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < kLoraWaves; ++w) v += red[w][t][i][lane];
            const int64_t m = m0 + 4 * lg + i;
            if (m < M) z[m * (16 * RT) + t * 16 + lr] = (uint16_t)f32_to_bf16_bits(v);
        }
    }
}

}  // namespace

namespace rq {

hipError_t launch_lora_down(const void* x, int64_t m, int64_t k, const void* a, int rank, void* z,
                            hipStream_t stream) {
    const int blocks = (int)((m + 15) / 16);
    if (blocks == 0) return hipSuccess;
    const dim3 grid(blocks);
    const uint16_t* xp = (const uint16_t*)x;
    const uint16_t* ap = (const uint16_t*)a;
    uint16_t* zp = (uint16_t*)z;
    switch (rank) {
        case 16: hipLaunchKernelGGL((lora_down_kernel<1>), grid, dim3(64 * LoraShape<1>::W), 0, stream, xp, m, k, ap, zp); break;
        case 32: hipLaunchKernelGGL((lora_down_kernel<2>), grid, dim3(64 * LoraShape<2>::W), 0, stream, xp, m, k, ap, zp); break;
        case 48: hipLaunchKernelGGL((lora_down_kernel<3>), grid, dim3(64 * LoraShape<3>::W), 0, stream, xp, m, k, ap, zp); break;
        case 64: hipLaunchKernelGGL((lora_down_kernel<4>), grid, dim3(64 * LoraShape<4>::W), 0, stream, xp, m, k, ap, zp); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rq
