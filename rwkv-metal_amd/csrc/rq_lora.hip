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
//  * AT: the adapter comes as its transpose b = a^T [K, rank] (row-major; the
//    QLoRA backward's B as the layer stores it, u = dY . B).  A k-step's 32
//    rows of b (rank * 64 bytes) are loaded as they lie, 16 bytes a lane, and
//    copied to the wave's own LDS buffer; each 16 x 32 fragment then comes
//    from two gfx950 ds_read_b64_tr_b16 (source lane 4 s + c of a 16-lane
//    group reads ranks 4 c .. +3 of row s).  The sums are the same as with a,
//    in the same order.
//  * XF: x is fp32; each 8-value chunk is loaded as 32 bytes and rounded to
//    bf16 (RNE) before its MFMA, so z equals the bf16(x) launch's bit for bit.
#include <mutex>

#include "rq_common.h"
#include "rq_launch.h"

namespace {

// waves per block and k-steps per batch of loads, by rank tiles: two
// register sets of U x (1 + RT) 16-byte loads stay within the VGPRs the
// block size allows (128 at 16 waves, 256 at 8; the a^T and fp32-x forms
// hold more per k-step and batch 2 at rank 16).  Wave w sums k-steps w,
// w + W, .. in order and the waves are summed in order, so the bits depend
// on W alone: the forms of one rank share it.
template <int RT, bool AT = false, bool XF = false> struct LoraShape {
    static constexpr int W = RT == 1 ? 16 : 8;
    static constexpr int U = (RT == 1 && (AT || XF)) ? 2 : (RT <= 2 ? 4 : 2);
};

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int RT, bool AT = false, bool XF = false>  // rank tiles of 16; AT: a given as
                                                    // a^T [K, rank]; XF: fp32 x
__global__ __launch_bounds__((64 * LoraShape<RT, AT, XF>::W)) void lora_down_kernel(
    const void* __restrict__ x, int64_t M, int64_t K, const uint16_t* __restrict__ a,
    uint16_t* __restrict__ z) {
    constexpr int kLoraWaves = LoraShape<RT, AT, XF>::W, U = LoraShape<RT, AT, XF>::U;
    constexpr int RANK = 16 * RT;
    __shared__ __attribute__((aligned(16))) float red[kLoraWaves][RT][4][64];
    __shared__ __attribute__((aligned(16))) uint8_t slab[AT ? kLoraWaves : 1][AT ? 64 * RANK : 16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lg = lane >> 4, lr = lane & 15;
    const int64_t m0 = (int64_t)blockIdx.x * 16;
    const int64_t row = (m0 + lr) < M ? (m0 + lr) : M - 1;  // rows past M: any valid row
    const int nsteps = (int)(K >> 5);
    constexpr int EB = XF ? 4 : 2;  // bytes per x element
    const uint8_t* xr = (const uint8_t*)x + (row * K + lg * 8) * EB;
    // a: this lane's fragment row; a^T: this lane's 16-byte chunks of a k-step's rows
    const uint16_t* ar = AT ? a + lane * 8 : a + (int64_t)lr * K + lg * 8;
    typedef short s16x4_t __attribute__((ext_vector_type(4)));
    typedef short s16x8_t __attribute__((ext_vector_type(8)));
    typedef __attribute__((address_space(3))) s16x4_t* lds_s16x4_p;
    uint8_t* wslab = slab[AT ? wave : 0];

    f32x4_t acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // Batches of U k-steps, software-pipelined: the loads of batch j + 1 are
    // issued before the MFMAs of batch j.  Loads past the end read the last
    // k-step (valid memory) and are not used.
    u32x4_t xa[2][U][XF ? 2 : 1], wb[2][U][RT];
    auto load = [&](int b, int s0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int s = s0 + kLoraWaves * u;
            s = s < nsteps ? s : nsteps - 1;
            const u32x4_t* xs = (const u32x4_t*)(xr + (int64_t)s * 32 * EB);
            xa[b][u][0] = xs[0];
            if constexpr (XF) xa[b][u][1] = xs[1];
#pragma unroll
            for (int t = 0; t < RT; ++t)
                wb[b][u][t] = AT ? *(const u32x4_t*)(ar + (int64_t)s * 32 * RANK + t * 512)
                                 : *(const u32x4_t*)(ar + ((int64_t)t * 16 * K + (int64_t)s * 32));
        }
    };
    auto mma = [&](int b, int s0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (s0 + kLoraWaves * u < nsteps) {
                u32x4_t xv = xa[b][u][0];
                if constexpr (XF) {
                    const u32x4_t p = xa[b][u][0], q = xa[b][u][1];
                    xv = u32x4_t{pack_bf16x2(__uint_as_float(p[0]), __uint_as_float(p[1])),
                                 pack_bf16x2(__uint_as_float(p[2]), __uint_as_float(p[3])),
                                 pack_bf16x2(__uint_as_float(q[0]), __uint_as_float(q[1])),
                                 pack_bf16x2(__uint_as_float(q[2]), __uint_as_float(q[3]))};
                }
                const bf16x8_t av = __builtin_bit_cast(bf16x8_t, xv);
                if constexpr (AT) {
                    // the k-step's rows of a^T into this wave's buffer (one wave's LDS
                    // operations complete in order: the reads below see these
                    // writes, and the next u's writes follow these reads)
                    asm volatile("" ::: "memory");
#pragma unroll
                    for (int t = 0; t < RT; ++t) *(u32x4_t*)(wslab + (lane + 64 * t) * 16) = wb[b][u][t];
                    asm volatile("" ::: "memory");
                }
#pragma unroll
                for (int t = 0; t < RT; ++t) {
                    bf16x8_t bv;
                    if constexpr (AT) {
                        // rows 8 lg + 4 v + lr / 4 of the k-step, ranks 16 t + 4 (lr % 4) .. +3
                        const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_p)(
                            wslab + (8 * lg + (lr >> 2)) * 2 * RANK + (16 * t + 4 * (lr & 3)) * 2));
                        const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_p)(
                            wslab + (8 * lg + 4 + (lr >> 2)) * 2 * RANK + (16 * t + 4 * (lr & 3)) * 2));
                        bv = __builtin_bit_cast(bf16x8_t,
                                                s16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
                    } else {
                        bv = __builtin_bit_cast(bf16x8_t, wb[b][u][t]);
                    }
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[t], 0, 0, 0);
                }
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

// ------------------------------------------------------------ lora_grads
//
// The QLoRA adapter gradients (MLX autograd of LoRALinear.__call__,
// rwkv_metal/lora/lora.py:58-63, through nn.value_and_grad at
// rwkv_metal/lora/finetune.py:141), both contractions over the M token rows:
//   dA[j, k] = scale * sum_m u[m, j] * x[m, k]      (u = dY . B, [M, rank])
//   dB[n, j] = scale * sum_m dY[m, n] * z[m, j]     (z = x . A^T, [M, rank])
// One launch covers both.  A job is a 64-column tile of x (dA) or dY (dB)
// times the rank over one chunk of the rows.  With S > 1 chunks per tile
// each chunk's fp32 partial tile goes to scratch memory and the chunk that
// finishes last (a per-tile counter) sums the S partials in chunk order,
// scales, rounds once to bf16, stores the tile and resets the counter to
// zero; with S = 1 the job stores its tile directly.  Deterministic: the
// same inputs give the same bits whatever order the chunks finish in.
//
// v_mfma_f32_16x16x32_bf16 contracts over 32 rows: A = 16 columns of wave
// w's 16-column slice (lane: column lr, rows 8 lg .. +7), B = 16 ranks (lane:
// rank lr, the same rows).  Both operands want the rows contiguous per lane
// while the tensors are row-major [M, *]: every 64-row step is written to
// LDS as it is, row-major, with 16-byte stores, and the fragments come from
// gfx950's transposing ds_read_b64_tr_b16 (within 16 lanes, source lane
// 4 s + a reads 4 columns 4 a .. +3 of row s, and result lane 4 a + b
// receives column 4 a + b of the 4 rows; two reads give a lane 8 rows).  The
// x / dY tile's 16-byte chunks are XOR-swizzled by 2 (row % 4), so the 4 rows
// x 2 chunks of one transposed read hit 8 different bank groups.  (The
// earlier layout, transposed in LDS by 2-byte stores, spent the step on
// those stores: 26.7 us per config-4 projection.)

constexpr int kGradBlock = 256;

RQ_DEV int pchunk(int c, int m) { return c ^ ((m & 3) << 1); }

template <int RT, bool PF>  // rank / 16; PF: x and dY are fp32 (rounded to bf16 as they are staged)
__global__ __launch_bounds__(kGradBlock) void lora_grads_kernel(
    const void* __restrict__ x, const uint16_t* __restrict__ u,
    const void* __restrict__ dy, const uint16_t* __restrict__ z, int64_t M, int64_t K,
    int64_t N, float scale, uint16_t* __restrict__ da, uint16_t* __restrict__ db,
    float* __restrict__ part, uint32_t* __restrict__ cnt, int tiles_a, int S, int64_t mchunk) {
    constexpr int RANK = 16 * RT;
    constexpr int QV = RANK * 64 / 8;            // 16-byte chunks of a 64-row step of Q
    constexpr int QL = (QV + kGradBlock - 1) / kGradBlock;
    __shared__ __attribute__((aligned(16))) uint16_t pt[2][64 * 64];    // [row][column], chunks swizzled
    __shared__ __attribute__((aligned(16))) uint16_t qt[2][64 * RANK];  // [row][rank]
    __shared__ uint32_t last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lg = lane >> 4, lr = lane & 15;
    const int tile = (int)(blockIdx.x / S), s = (int)(blockIdx.x % S);
    const bool is_a = tile < tiles_a;
    const uint8_t* P = (const uint8_t*)(is_a ? x : dy);
    constexpr int PB = PF ? 4 : 2;  // bytes per x / dY element
    const uint16_t* Q = is_a ? u : z;
    const int64_t C = is_a ? K : N;
    const int64_t c0 = (int64_t)(is_a ? tile : tile - tiles_a) * 64;
    const int64_t mb = (int64_t)s * mchunk;
    const int64_t me = M < mb + mchunk ? M : mb + mchunk;
    const int nsteps = (int)((me - mb + 63) / 64);

    // thread t loads rows t / 8 and t / 8 + 32 of the 64-column tile, columns
    // 8 (t % 8) .. +7 (C % 8 == 0: a chunk is wholly inside or outside)
    const int prow = tid >> 3, pch = tid & 7;
    const bool pcol = c0 + pch * 8 < C;
    u32x4_t pv[2][PF ? 2 : 1], qv[QL];
    auto load = [&](int st) {
        const int64_t m = mb + (int64_t)st * 64;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t r = m + prow + 32 * h;
#pragma unroll
            for (int e = 0; e < (PF ? 2 : 1); ++e) pv[h][e] = u32x4_t{0u, 0u, 0u, 0u};
            if (r < me && pcol) {
                const u32x4_t* src = (const u32x4_t*)(P + (r * C + c0 + pch * 8) * PB);
                pv[h][0] = src[0];
                if constexpr (PF) pv[h][1] = src[1];
            }
        }
#pragma unroll
        for (int i = 0; i < QL; ++i) {
            const int q = tid + kGradBlock * i;
            qv[i] = u32x4_t{0u, 0u, 0u, 0u};
            if (QV % kGradBlock == 0 || q < QV) {
                const int64_t r = m + q / (RANK / 8);
                if (r < me) qv[i] = *(const u32x4_t*)(Q + r * RANK + (q % (RANK / 8)) * 8);
            }
        }
    };
    auto put = [&](int b) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int m = prow + 32 * h;
            u32x4_t v = pv[h][0];
            if constexpr (PF)
                v = u32x4_t{pack_bf16x2(__uint_as_float(pv[h][0][0]), __uint_as_float(pv[h][0][1])),
                            pack_bf16x2(__uint_as_float(pv[h][0][2]), __uint_as_float(pv[h][0][3])),
                            pack_bf16x2(__uint_as_float(pv[h][1][0]), __uint_as_float(pv[h][1][1])),
                            pack_bf16x2(__uint_as_float(pv[h][1][2]), __uint_as_float(pv[h][1][3]))};
            *(u32x4_t*)(pt[b] + m * 64 + pchunk(pch, m) * 8) = v;
        }
#pragma unroll
        for (int i = 0; i < QL; ++i) {
            const int q = tid + kGradBlock * i;
            if (QV % kGradBlock == 0 || q < QV) *(u32x4_t*)(qt[b] + q * 8) = qv[i];
        }
    };

    f32x4_t acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // transposed-read source addresses (elements): row 8 lg + 4 v + lr / 4 of
    // the 32-row k-step, columns 4 (lr % 4) .. +3 of the 16-wide slice
    typedef short s16x4_t __attribute__((ext_vector_type(4)));
    typedef short s16x8_t __attribute__((ext_vector_type(8)));
    typedef __attribute__((address_space(3))) s16x4_t* lds_s16x4_p;
    uint32_t aoff[2], boff[2];
#pragma unroll
    for (int v = 0; v < 2; ++v) {
        const int row = 8 * lg + 4 * v + (lr >> 2);
        const int col = 16 * wave + 4 * (lr & 3);
        aoff[v] = (uint32_t)(row * 64 + pchunk(col >> 3, row) * 8 + (col & 7));
        boff[v] = (uint32_t)(row * RANK + 4 * (lr & 3));
    }
    auto tread = [&](const uint16_t* base) {
        return (lds_s16x4_p)(base);
    };
    if (nsteps > 0) load(0);
    for (int st = 0; st < nsteps; ++st) {
        const int b = st & 1;
        put(b);
        if (st + 1 < nsteps) load(st + 1);  // in flight across the barrier and the MFMAs
        // own LDS writes (and the previous step's reads of the other buffer) done
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            // rows 32 ks .. : the swizzle key depends on row % 4 only
            const s16x4_t a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(tread(pt[b] + aoff[0] + ks * 32 * 64));
            const s16x4_t a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(tread(pt[b] + aoff[1] + ks * 32 * 64));
            const bf16x8_t av = __builtin_bit_cast(
                bf16x8_t, s16x8_t{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]});
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                const s16x4_t b0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    tread(qt[b] + boff[0] + ks * 32 * RANK + 16 * t));
                const s16x4_t b1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    tread(qt[b] + boff[1] + ks * 32 * RANK + 16 * t));
                const bf16x8_t bv = __builtin_bit_cast(
                    bf16x8_t, s16x8_t{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]});
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[t], 0, 0, 0);
            }
        }
    }

    // lane (lg, lr) of wave w holds acc[t][i]: column 16 w + 4 lg + i, rank 16 t + lr
    uint16_t* out = is_a ? da : db;
    auto store = [&](int c, int j, float v) {
        if (c0 + c >= C) return;
        const int64_t o = is_a ? (int64_t)j * K + c0 + c : (c0 + c) * RANK + j;
        out[o] = (uint16_t)f32_to_bf16_bits(scale * v);
    };
    if (S == 1) {
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) store(16 * wave + 4 * lg + i, 16 * t + lr, acc[t][i]);
        return;
    }
    // The partial tiles cross XCDs, whose L2s are not coherent with each other.
    // They are written and read back with relaxed agent-scope atomic stores
    // and loads, which are coherent across the device by themselves, so no
    // agent-scope fence is needed (on gfx950 each would write back or
    // invalidate the whole L2 of the XCD: ~100 us per launch at ~1000 jobs).
    // Every thread waits for its stores to complete before the block counts
    // itself in; the last chunk to count reads the others' tiles.
    float* mine = part + ((int64_t)tile * S + s) * (64 * RANK);
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __hip_atomic_store(mine + (16 * wave + 4 * lg + i) * RANK + 16 * t + lr, acc[t][i],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (uint32_t)(S - 1);
    __syncthreads();
    if (!last) return;
    // the S partials of this thread's elements, summed in chunk order; the
    // loads go out QB chunks at a time, 64 values per thread (one at a time,
    // each waiting for the previous sum, they made the reduction a chain of S
    // memory latencies: 27.5 vs 15.0 us per config-4 r/k/v/o launch)
    const float* tp = part + (int64_t)tile * S * (64 * RANK);
    constexpr int EPT = 64 * RANK / kGradBlock;  // elements per thread
    constexpr int QB = 64 / EPT;                 // chunks per batch of loads
    static_assert(EPT * kGradBlock == 64 * RANK, "");
    float v[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i) v[i] = 0.f;
    for (int q0 = 0; q0 < S; q0 += QB) {
        float t[QB][EPT];
#pragma unroll
        for (int j = 0; j < QB; ++j)
#pragma unroll
            for (int i = 0; i < EPT; ++i)
                t[j][i] = q0 + j < S ? __hip_atomic_load(tp + (int64_t)(q0 + j) * (64 * RANK) + tid +
                                                             kGradBlock * i,
                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                     : 0.f;
#pragma unroll
        for (int j = 0; j < QB; ++j)
#pragma unroll
            for (int i = 0; i < EPT; ++i)
                if (q0 + j < S) v[i] += t[j][i];
    }
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int e = tid + kGradBlock * i;
        store(e / RANK, e % RANK, v[i]);
    }
    if (tid == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void zero_words_kernel(uint32_t* __restrict__ p, int n) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) p[i] = 0u;
}

// The no-allocation form's work buffer: counters and fp32 partial tiles of
// the gradient launch, one copy per GPU, held until the process ends.  Host
// code never uses this name as an address (it is a host-side stand-in): the
// device address comes from hipGetSymbolAddress, per device.
static __device__ __align__(256) uint8_t scratch[rq::kLoraScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
bool g_scratch_zeroed[kMaxDevices] = {};

}  // namespace

namespace rq {

hipError_t lora_scratch(void** out, hipStream_t stream) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[dev] = p;
    }
    if (!g_scratch_zeroed[dev]) {
        // the counters must start at zero (each launch leaves them so); a fill
        // kernel rather than a memset node, so the stream may be capturing.
        // Launched into a graph being captured it runs only when the graph is
        // replayed (before that graph's own gradient launch), so the device
        // counts as cleared only after an eager clear.
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(stream, &cap);
        if (e != hipSuccess) return e;
        const int words = (int)(kLoraGradCounterBytes / 4);
        hipLaunchKernelGGL(zero_words_kernel, dim3((words + 255) / 256), dim3(256), 0, stream,
                           (uint32_t*)g_scratch_ptr[dev], words);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (cap == hipStreamCaptureStatusNone) g_scratch_zeroed[dev] = true;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

LoraGradPlan lora_grads_plan(int64_t m, int64_t k, int64_t n, int rank, bool has_a, bool has_b) {
    LoraGradPlan p;
    p.tiles_a = has_a ? (int)((k + 63) / 64) : 0;
    p.tiles_b = has_b ? (int)((n + 63) / 64) : 0;
    const int64_t tiles = p.tiles_a + p.tiles_b;
    const int64_t steps = (m + 63) / 64;
    int64_t S = tiles > 0 ? (kLoraGradTargetBlocks + tiles - 1) / tiles : 1;
    S = S < steps ? S : steps;
    const int64_t per_split = tiles * 64 * (int64_t)rank * 4;
    if (per_split > 0 && S * per_split > kLoraGradPartialCap) S = kLoraGradPartialCap / per_split;
    if (S < 1) S = 1;
    const int64_t per = (steps + S - 1) / S;  // 64-row steps per chunk
    p.mchunk = per * 64;
    p.splits = steps > 0 ? (int)((steps + per - 1) / per) : 1;
    p.partial_bytes = p.splits > 1 ? (size_t)(tiles * p.splits * 64 * (int64_t)rank * 4) : 0;
    p.work_bytes = p.splits > 1 ? kLoraGradCounterBytes + p.partial_bytes : 0;
    return p;
}

hipError_t launch_lora_grads(const void* x, const void* u, const void* dy, const void* z,
                             int64_t m, int64_t k, int64_t n, int rank, float scale, void* da,
                             void* db, const LoraGradPlan& p, void* work, hipStream_t stream,
                             bool xdy_f32) {
    const int tiles = p.tiles_a + p.tiles_b;
    if (tiles == 0) return hipSuccess;
    uint32_t* cnt = (uint32_t*)work;
    float* part = (float*)((uint8_t*)work + kLoraGradCounterBytes);
    const dim3 grid((unsigned)(tiles * p.splits)), block(kGradBlock);
    const uint16_t *up = (const uint16_t*)u, *zp = (const uint16_t*)z;
    uint16_t *dap = (uint16_t*)da, *dbp = (uint16_t*)db;
#define RQ_GRADS(RT)                                                                           \
    if (xdy_f32)                                                                               \
        hipLaunchKernelGGL((lora_grads_kernel<RT, true>), grid, block, 0, stream, x, up, dy, zp,  \
                           m, k, n, scale, dap, dbp, part, cnt, p.tiles_a, p.splits, p.mchunk);  \
    else                                                                                       \
        hipLaunchKernelGGL((lora_grads_kernel<RT, false>), grid, block, 0, stream, x, up, dy, zp, \
                           m, k, n, scale, dap, dbp, part, cnt, p.tiles_a, p.splits, p.mchunk)
    switch (rank) {
        case 16: RQ_GRADS(1); break;
        case 32: RQ_GRADS(2); break;
        case 48: RQ_GRADS(3); break;
        case 64: RQ_GRADS(4); break;
        default: return hipErrorInvalidValue;
    }
#undef RQ_GRADS
    return hipGetLastError();
}

hipError_t launch_lora_down(const void* x, int64_t m, int64_t k, const void* a, int rank, void* z,
                            hipStream_t stream, bool a_t, bool x_f32) {
    const int blocks = (int)((m + 15) / 16);
    if (blocks == 0) return hipSuccess;
    const dim3 grid(blocks);
    const uint16_t* ap = (const uint16_t*)a;
    uint16_t* zp = (uint16_t*)z;
#define RQ_DOWN_X(RT, ATV)                                                                         \
    if (x_f32)                                                                                     \
        hipLaunchKernelGGL((lora_down_kernel<RT, ATV, true>), grid,                                \
                           dim3(64 * LoraShape<RT, ATV, true>::W), 0, stream, x, m, k, ap, zp);    \
    else                                                                                           \
        hipLaunchKernelGGL((lora_down_kernel<RT, ATV, false>), grid,                               \
                           dim3(64 * LoraShape<RT, ATV, false>::W), 0, stream, x, m, k, ap, zp);
#define RQ_DOWN(RT)                                                                                \
    if (a_t) {                                                                                     \
        RQ_DOWN_X(RT, true)                                                                        \
    } else {                                                                                       \
        RQ_DOWN_X(RT, false)                                                                       \
    }
    switch (rank) {
        case 16: RQ_DOWN(1) break;
        case 32: RQ_DOWN(2) break;
        case 48: RQ_DOWN(3) break;
        case 64: RQ_DOWN(4) break;
        default: return hipErrorInvalidValue;
    }
#undef RQ_DOWN
#undef RQ_DOWN_X
    return hipGetLastError();
}

}  // namespace rq
