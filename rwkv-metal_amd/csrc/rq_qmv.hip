// rq_qmv.hip -- decode GEMV for group-affine packed weights (gfx950).
//
//   y[m, r] = sum_k x[m, k] * (scale[r, g(k)] * code[r, k] + bias[r, g(k)]),  m <= 16
//
// This is mx.quantized_matmul(transpose=True) at decode sizes, reached from
// QuantizedLinear / LoRALinear.__call__ (rwkv_metal/lora/lora.py:58-59) and the
// decode path of the model (rwkv_metal/model/rwkv7_x070.py:174-182, head :343).
//
// Design.  The kernel is HBM-bound: every packed weight byte is read once.
// The multiply by x runs on the matrix cores so that the VALU only turns
// packed codes into bf16 operands, which is what limits a plain VALU GEMV:
//
//  * v_mfma_f32_16x16x32_bf16 with A = activations (16 rows m'), B = weight
//    codes (16 weight rows n, 32 codes each), D[m'][n].  Lane L supplies
//    B[8(L/16)..+7][L%16]: eight codes of weight row L%16 -- and receives
//    D[4(L/16)+i][L%16], i.e. outputs of that same weight row.  So each lane
//    needs only the scale and bias of its own row and its own run's group.
//  * A "span" is 4 runs (128 codes) of 16 rows.  Lane L loads run (L/16) of
//    the span for row L%16 with one 128-bit load (4-bit) -- 16 rows x 64 B
//    contiguous per wave-load.  MFMA j (j=0..3) consumes word j of every
//    lane's run; the contraction order inside an MFMA is irrelevant as long
//    as A uses the same order.
//  * Codes become bf16 without a convert: (128 + q) has bf16 bits 0x4300|q
//    for q < 128, so ((w >> 4i) & 0x000F000F) | 0x43004300 yields codes
//    (i, i+4) of a 4-bit word as two bf16 in one v_and_or.  A holds x in
//    the matching order (x_i, x_{i+4}).
//  * A span can hold several groups ("slots": 4 at gs=32, 2 at gs=64, 1 at
//    gs=128).  The 16 A rows are split into slots: A row m' carries x[m]
//    only for the runs of slot m'/MC (MC = 16/slots) and zero elsewhere,
//    so D row m' sums exactly one group and the lane's per-row scale can be
//    applied to it.  M up to MC per pass; larger M uses NMC passes that
//    share the loaded codes.
//  * The +128 offset is removed with a second MFMA per span on a constant
//    B (all 128.0): O[m'][n] = 128 * sum_{k in slot} x[m][k], in the same
//    accumulator layout as D.  Then
//        acc += s * D + (b/128 - s) * O  ==  s * sum q x + b * sum x.
//    8-bit codes use exact bf16(q) operands (q <= 255 has 8 significant
//    bits) and a constant B of 1.0.
//  * A block of 4 waves owns 16*RB rows; the waves split the spans of K and
//    their partial sums meet in LDS at the end.  One launch can cover many
//    independent problems (rq_qmm_grouped): each block looks its problem up
//    in a prefix table of block counts.
#include "rq_common.h"
#include "rq_launch.h"

#include <cstring>

#ifndef RQ_BITS
#error "compile rq_qmv.hip once per bit width with -DRQ_BITS=<bits>"
#endif

namespace {

constexpr int kWaves = 4;
constexpr int kBlock = 64 * kWaves;

struct QmvArgs {
    rq_problem p[RQ_MAX_GROUPED];
    int block_start[RQ_MAX_GROUPED + 1];
    int n;
    int m;
    int gs_shift;
    int sb_dt;
    int y_dt;
};

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

RQ_DEV bf16x8_t as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4_t v = {a, b, c, d};
    return __builtin_bit_cast(bf16x8_t, v);
}

// Eight codes 8j..8j+7 of a run as bf16 pairs (c_i, c_{i+4}), i = 0..3.
template <int BITS>
RQ_DEV void codes_to_bf16_pairs(const uint32_t* words, int j, uint32_t* out) {
    if constexpr (BITS == 4) {
        const uint32_t w = words[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = ((w >> (4 * i)) & 0x000F000Fu) | 0x43004300u;
    } else if constexpr (BITS == 8) {
        const uint32_t lo = words[2 * j], hi = words[2 * j + 1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // v_cvt_f32_ubyte<i>; the high halves are exact bf16(q)
            const float fl = (float)((lo >> (8 * i)) & 0xffu);
            const float fh = (float)((hi >> (8 * i)) & 0xffu);
            out[i] = __builtin_amdgcn_perm(__float_as_uint(fh), __float_as_uint(fl), 0x07060302u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            out[i] = run_code<BITS>(words, 8 * j + i) |
                     (run_code<BITS>(words, 8 * j + i + 4) << 16) | 0x43004300u;
    }
}

// Eight activations x[8j..8j+7] (as 4 dwords of bf16 pairs in natural order
// n0=(x0,x1) n1=(x2,x3) n2=(x4,x5) n3=(x6,x7)) -> pairs (x_i, x_{i+4}).
RQ_DEV void reorder_pairs(const uint32_t* n, uint32_t* out) {
    out[0] = __builtin_amdgcn_perm(n[2], n[0], 0x05040100u);
    out[1] = __builtin_amdgcn_perm(n[2], n[0], 0x07060302u);
    out[2] = __builtin_amdgcn_perm(n[3], n[1], 0x05040100u);
    out[3] = __builtin_amdgcn_perm(n[3], n[1], 0x07060302u);
}

// Load the 32 activations of one run of row m as 16 bf16-pair dwords.
template <int XDT>
RQ_DEV void load_x_run_bf16(const void* x, int64_t off, uint32_t* d) {
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
}

template <int BITS, int XDT, int NMC, int RB>
__global__ __launch_bounds__(kBlock) void qmv_kernel(const QmvArgs args) {
    const int bid = blockIdx.x;
    int p = 0;
    while (p + 1 < args.n && args.block_start[p + 1] <= bid) ++p;
    const void* __restrict__ x = args.p[p].x;
    const uint32_t* __restrict__ wq = args.p[p].w_q;
    const void* __restrict__ scales = args.p[p].scales;
    const void* __restrict__ biases = args.p[p].biases;
    const int64_t R = args.p[p].rows;
    const int64_t K = args.p[p].cols;
    const int64_t row0 = (int64_t)(bid - args.block_start[p]) * (16 * RB);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int lg = lane >> 4;  // lane group: run inside the span / k-slice
    const int lr = lane & 15;  // A row m' / weight row inside a 16-row block
    const int M = args.m;
    const int gsh = args.gs_shift;
    const int slot_shift = gsh - 5;  // run index -> group index
    const int MC = 16 >> (7 - gsh);  // activation rows per pass
    const int sb_dt = args.sb_dt;

    const int64_t runs_per_row = K >> 5;
    const int64_t wpr = runs_per_row * BITS;  // packed words per row
    const int64_t G = K >> gsh;
    const int nspans = (int)((runs_per_row + 3) >> 2);

    // A-side role of this lane: activation row (per pass) and slot.
    const bool a_slot_ok = (lr / MC) == (lg >> slot_shift);

    constexpr uint32_t kOne = (BITS == 8) ? 0x3F803F80u : 0x43004300u;  // 1.0 or 128.0
    const bf16x8_t ones = as_bf16x8(kOne, kOne, kOne, kOne);

    f32x4_t acc[RB][NMC];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int c = 0; c < NMC; ++c) acc[rb][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int s = wave; s < nspans; s += kWaves) {
        const int64_t run = (int64_t)s * 4 + lg;
        const bool run_ok = run < runs_per_row;

        // B side: this lane's run of its row in every row block.
        uint32_t cw[RB][BITS];
        float sc[RB], bi[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int64_t row = row0 + rb * 16 + lr;
            if (run_ok && row < R) {
                load_run<BITS>(wq + row * wpr + run * BITS, cw[rb]);
                const int64_t gi = row * G + (run >> slot_shift);
                sc[rb] = load_dt(scales, sb_dt, gi);
                bi[rb] = load_dt(biases, sb_dt, gi);
            } else {
#pragma unroll
                for (int w = 0; w < BITS; ++w) cw[rb][w] = 0u;
                sc[rb] = 0.f;
                bi[rb] = 0.f;
            }
        }

        // A side: activations of this lane's run for each pass.
        bf16x8_t a[NMC][4];
        f32x4_t o[NMC];
#pragma unroll
        for (int c = 0; c < NMC; ++c) {
            const int m = c * MC + (lr % MC);
            uint32_t xd[16];
            if (a_slot_ok && run_ok && m < M) {
                load_x_run_bf16<XDT>(x, (int64_t)m * K + run * 32, xd);
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) xd[i] = 0u;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t pr[4];
                reorder_pairs(&xd[4 * j], pr);
                a[c][j] = as_bf16x8(pr[0], pr[1], pr[2], pr[3]);
            }
            o[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                o[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[c][j], ones, o[c], 0, 0, 0);
        }

#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            bf16x8_t bop[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t pr[4];
                codes_to_bf16_pairs<BITS>(cw[rb], j, pr);
                bop[j] = as_bf16x8(pr[0], pr[1], pr[2], pr[3]);
            }
            const float cb = (BITS == 8) ? bi[rb] : (bi[rb] * 0.0078125f - sc[rb]);
#pragma unroll
            for (int c = 0; c < NMC; ++c) {
                f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[c][j], bop[j], d, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[rb][c][i] = fmaf(sc[rb], d[i], fmaf(cb, o[c][i], acc[rb][c][i]));
            }
        }
    }

    // Cross-wave sum and slot combine through LDS.
    __shared__ float red[kWaves][RB][NMC][4][64];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int c = 0; c < NMC; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][rb][c][i][lane] = acc[rb][c][i];
    __syncthreads();

    const int slots = 1 << (7 - gsh);
    const int total = RB * 16 * M;
    for (int idx = threadIdx.x; idx < total; idx += kBlock) {
        const int rb = idx / (16 * M);
        const int rem = idx - rb * 16 * M;
        const int m = rem >> 4;
        const int n = rem & 15;
        const int c = m / MC;
        const int mm = m - c * MC;
        float sum = 0.f;
        for (int sl = 0; sl < slots; ++sl) {
            const int mp = sl * MC + mm;  // D row
            const int L = n + 16 * (mp >> 2);
            const int i = mp & 3;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) sum += red[w][rb][c][i][L];
        }
        const int64_t row = row0 + rb * 16 + n;
        if (row < R) store_dt(args.p[p].y, args.y_dt, (int64_t)m * R + row, sum);
    }
}

template <int XDT, int NMC, int RB>
hipError_t launch_one(const QmvArgs& a, int blocks, hipStream_t stream) {
    hipLaunchKernelGGL((qmv_kernel<RQ_BITS, XDT, NMC, RB>), dim3(blocks), dim3(kBlock), 0, stream,
                       a);
    return hipGetLastError();
}

template <int RB>
hipError_t launch_rb(const QmvArgs& a, int x_dt, int nmc, int blocks, hipStream_t stream) {
    hipError_t e = hipErrorInvalidValue;
    RQ_DISPATCH_DT(x_dt, XD,
        switch (nmc) {
            case 1: e = launch_one<XD, 1, RB>(a, blocks, stream); break;
            case 2: e = launch_one<XD, 2, RB>(a, blocks, stream); break;
            case 4: e = launch_one<XD, 4, RB>(a, blocks, stream); break;
            default: break;
        });
    return e;
}

}  // namespace

namespace rq {

#define RQ_CAT2(a, b) a##b
#define RQ_CAT(a, b) RQ_CAT2(a, b)

hipError_t RQ_CAT(launch_qmv_b, RQ_BITS)(const rq_problem* problems, int n, int x_dt, int sb_dt,
                                         int y_dt, int64_t m, int gs, hipStream_t stream) {
    const int gs_shift = __builtin_ctz(gs);
    const int MC = 16 >> (7 - gs_shift);
    int nmc = (int)((m + MC - 1) / MC);
    nmc = nmc <= 1 ? 1 : (nmc <= 2 ? 2 : 4);

    // Total 16-row blocks decide the rows per block: a launch that can keep
    // every CU busy with 64-row blocks uses them (fewer partial-sum meets),
    // smaller launches use 16-row blocks for parallelism.
    int64_t rowblocks = 0;
    for (int i = 0; i < n; ++i) rowblocks += (problems[i].rows + 15) / 16;
    const int RB = rowblocks >= 4096 ? 4 : 1;

    for (int base = 0; base < n; base += RQ_MAX_GROUPED) {
        const int cnt = (n - base) < RQ_MAX_GROUPED ? (n - base) : RQ_MAX_GROUPED;
        QmvArgs a;
        std::memset(&a, 0, sizeof(a));
        int64_t blocks = 0;
        for (int i = 0; i < cnt; ++i) {
            a.p[i] = problems[base + i];
            a.block_start[i] = (int)blocks;
            blocks += (problems[base + i].rows + 16 * RB - 1) / (16 * RB);
        }
        a.block_start[cnt] = (int)blocks;
        a.n = cnt;
        a.m = (int)m;
        a.gs_shift = gs_shift;
        a.sb_dt = sb_dt;
        a.y_dt = y_dt;
        if (blocks == 0) continue;
        hipError_t e = RB == 4 ? launch_rb<4>(a, x_dt, nmc, (int)blocks, stream)
                               : launch_rb<1>(a, x_dt, nmc, (int)blocks, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace rq
