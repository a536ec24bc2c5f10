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
//  * The +128 offset is removed with the per-group sums of the activations,
//    X[m][g] = sum_{k in g} x[m][k], computed once per block while x is
//    staged (in LDS next to it):
//        acc += s * D + (b - 128 s) * X  ==  s * sum q x + b * sum x.
//    8-bit codes use exact bf16(q) operands (q <= 255 has 8 significant
//    bits) and acc += s * D + b * X.  Without LDS staging the sums come from
//    a second MFMA per span on a constant B (all 128.0, or 1.0 at 8 bits).
//  * A lane's accumulator holds D rows m' = 4*(lane/16) + i; at small M only
//    i < MI can be a real activation row (MI = min(M, 4) rounded up to a
//    power of two), so only those are updated and stored.
//  * Work unit ("task") = 16*RB rows of one problem.  A block of 4 waves
//    takes 4 consecutive tasks of one problem (KS=1, each wave walks every
//    span of K for its own rows) or, for small launches, one task whose
//    spans the 4 waves split and sum in LDS (KS=4).
//  * The activation rows x[0..M) of the block's problem are staged once in
//    LDS as bf16; A operands are read from there for every span, so only
//    packed codes (and their scales) live in registers: a wave issues the
//    loads of NS spans at once and consumes them in order.
//    When M*K*2 bytes exceed the LDS budget, A comes from global memory.
//  * One launch can cover many independent problems (rq_qmm_grouped): a
//    block finds its problem by binary search in a prefix table of block
//    counts held in the kernel arguments.
//
// The kernels: qmv_kernel (above: any layout), and for 16-bit scales the
// streamed qmv_stream_* (m <= 4) and qmv_wide_* (4 < m <= 16) for launches
// that fill the GPU with rows, and qmv_split for small launches (m <= 8; one
// memory round trip per launch); each is described where it is defined.

#include "rq_common.h"
#include "rq_launch.h"

#include <cstring>
#include <vector>
#include <type_traits>

#ifndef RQ_BITS
#error "compile rq_qmv.hip once per bit width with -DRQ_BITS=<bits>"
#endif

namespace {

constexpr int kWaves = 4;
constexpr int kBlock = 64 * kWaves;

// Compile-time tuning constants (overridable with -D for side-by-side builds).
#ifndef RQ_QMV_NS
#define RQ_QMV_NS 4  // rolling pipeline stages (LDS-staged path): NS-1 spans in flight
#endif
#ifndef RQ_QMV_BATCH
#define RQ_QMV_BATCH 8  // spans per batch on the global-scale path
#endif
#ifndef RQ_QMV_WAVES_PER_EU
#define RQ_QMV_WAVES_PER_EU 0  // >0: ask the compiler for this occupancy
#endif
#ifndef RQ_QMV_BIG_RB
#define RQ_QMV_BIG_RB 1  // 16-row blocks per wave for big launches
#endif
#ifndef RQ_QMV_WIDE
#define RQ_QMV_WIDE 1  // 0: never use the wide GEMV (4 < m <= 16)
#endif
#ifndef RQ_QMV_STREAM
#define RQ_QMV_STREAM 1  // 0: never use the streamed-scale GEMV
#endif
#ifndef RQ_QMV_SPLIT
#define RQ_QMV_SPLIT 1  // 0: never use the split GEMV (small launches)
#endif
#ifndef RQ_QMV_BIG_MIN
#define RQ_QMV_BIG_MIN 16384  // 16-row blocks in a launch from which RQ_QMV_BIG_RB applies
#endif
#if RQ_QMV_WAVES_PER_EU > 0
#define RQ_QMV_OCC __attribute__((amdgpu_waves_per_eu(RQ_QMV_WAVES_PER_EU)))
#else
#define RQ_QMV_OCC
#endif

struct QmvArgs {
    rq_problem p[RQ_MAX_GROUPED];
    int block_start[RQ_MAX_GROUPED + 1];  // prefix sums of blocks per problem
    int n;
    int m;
    int gs_shift;
    int x_dt;
    int y_dt;
    int sb_vec;  // scales and biases are 16-byte aligned (vector staging allowed)
    int xsplit;  // m counts the hi and lo bf16 rows of m/2 activation rows (qmv_xsplit)
    int fold;    // qmv_split: rows 2r, 2r + 1 are the halves of weight row r (split_fold)
};

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

RQ_DEV bf16x8_t as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4_t v = {a, b, c, d};
    return __builtin_bit_cast(bf16x8_t, v);
}

// Eight codes 8j..8j+7 of a run as bf16 pairs (c_i, c_{i+4}), i = 0..3.
// The mask and the bf16 exponent bits are passed in registers (opaque to the
// optimiser) so that each pair is one v_and_or_b32 instead of an and plus an
// or with literal operands.
struct PairConsts {
    uint32_t mask, magic;
};
RQ_DEV PairConsts pair_consts() {
    PairConsts c{0x000F000Fu, 0x43004300u};
    asm volatile("" : "+v"(c.mask), "+v"(c.magic));
    return c;
}

template <int BITS>
RQ_DEV void codes_to_bf16_pairs(const uint32_t* words, int j, uint32_t* out,
                                PairConsts k = PairConsts{0x000F000Fu, 0x43004300u}) {
    if constexpr (BITS == 4) {
        const uint32_t w = words[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = ((w >> (4 * i)) & k.mask) | k.magic;
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

// The second part of the hi/lo split of two activations: bf16(a - bf16(a))
// (the difference is exact in fp32).
RQ_DEV uint32_t pair_lo(float a, float b) {
    const uint32_t h = pack_bf16x2(a, b);
    return pack_bf16x2(a - __uint_as_float(h << 16), b - __uint_as_float(h & 0xffff0000u));
}

// The lo parts of the split of the 32 fp32 or f16 activations of one run.
RQ_DEV void load_x_run_lo(const void* x, int x_dt, int64_t off, uint32_t* d) {
    float f[32];
    if (x_dt == RQ_F32) load32_f32<RQ_F32>(x, off, f);
    else load32_f32<RQ_F16>(x, off, f);
#pragma unroll
    for (int i = 0; i < 16; ++i) d[i] = pair_lo(f[2 * i], f[2 * i + 1]);
}

// Streaming load of one run of packed codes.
#ifndef RQ_QMV_NT
#define RQ_QMV_NT 0  // 1: non-temporal code loads (measured: ~20% of lines fetched twice)
#endif
template <typename T>
RQ_DEV T ld_code(const T* p) {
#if RQ_QMV_NT
    return __builtin_nontemporal_load(p);
#else
    return *p;
#endif
}
template <int BITS>
RQ_DEV void load_run_stream(const uint32_t* p, uint32_t* words) {
    if constexpr (BITS == 4) {
        const u32x4_t v = ld_code((const u32x4_t*)p);
        words[0] = v[0]; words[1] = v[1]; words[2] = v[2]; words[3] = v[3];
    } else if constexpr (BITS == 8) {
        const u32x4_t v0 = ld_code((const u32x4_t*)p);
        const u32x4_t v1 = ld_code((const u32x4_t*)p + 1);
        words[0] = v0[0]; words[1] = v0[1]; words[2] = v0[2]; words[3] = v0[3];
        words[4] = v1[0]; words[5] = v1[1]; words[6] = v1[2]; words[7] = v1[3];
    } else {
#pragma unroll
        for (int w = 0; w < BITS; ++w) words[w] = ld_code(p + w);
    }
}

template <int BITS, int RB>
struct Stage {
    uint32_t cw[RB][BITS];   // this lane's run of its row, per row block
    uint32_t sc[RB], bi[RB];  // raw bits of that run's scale and bias (global-scale path)
};

// Raw bits of element i of a scales/biases array of dtype SDT.
template <int SDT>
RQ_DEV uint32_t load_raw(const void* p, int64_t i) {
    if constexpr (SDT == RQ_F32) return ((const uint32_t*)p)[i];
    else return ((const uint16_t*)p)[i];
}
template <int SDT>
RQ_DEV float raw_to_f32(uint32_t r) {
    if constexpr (SDT == RQ_F32) return __uint_as_float(r);
    else if constexpr (SDT == RQ_BF16) return bf16_bits_to_f32(r);
    else return f16_bits_to_f32(r & 0xffffu);
}

// One (scale, bias) pair as staged in LDS: two 16-bit values in one dword,
// or two fp32 values.
template <int SDT>
struct SBPair {
    typedef typename std::conditional<SDT == RQ_F32, uint2, uint32_t>::type type;
};

constexpr int kLdsBudget = rq::kQmvLdsBudget;  // bytes of LDS staging per block

// SLDS=true (fast path): the block's activations AND its rows' scales/biases
// are staged in LDS once; the span loop then streams only packed codes, with
// a rolling NS-stage register pipeline (NS-1 spans always in flight).
// SLDS=false (large M*K or K): activations and scales come from global
// memory; spans are processed in batches of NS (all loads of a batch issued
// first).  In both, loads are never predicated: out-of-range rows and runs
// read clamped, in-bounds addresses and are neutralised at compute time by a
// zero scale and bias (s*D + (b/128 - s)*O = 0).
template <int BITS, int SDT, int NMC, int MI, int RB, int KS, int NS, bool SLDS>
__global__ __launch_bounds__(kBlock) RQ_QMV_OCC void qmv_kernel(const QmvArgs args) {
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    typedef typename SBPair<SDT>::type sbp_t;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int bid = blockIdx.x;
    int lo = 0, hi = args.n - 1;  // last problem whose first block <= bid
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (args.block_start[mid] <= bid) lo = mid; else hi = mid - 1;
    }
    const int p = lo;
    const void* __restrict__ x = args.p[p].x;
    const uint32_t* __restrict__ wq = args.p[p].w_q;
    const void* __restrict__ scales = args.p[p].scales;
    const void* __restrict__ biases = args.p[p].biases;
    const int64_t R = args.p[p].rows;
    const int64_t K = args.p[p].cols;
    const int M = args.m;
    const int x_dt = args.x_dt;
    const int gsh = args.gs_shift;
    const int64_t G = K >> gsh;
    const int64_t lblock = bid - args.block_start[p];
    constexpr int kRowsPerBlock = (KS == 1 ? kWaves : 1) * 16 * RB;
    const int64_t blk_row0 = lblock * kRowsPerBlock;
    const int64_t row0 = blk_row0 + (KS == 1 ? wave * 16 * RB : 0);


    const int lg = lane >> 4;  // lane group: run inside the span / k-slice
    const int lr = lane & 15;  // A row m' / weight row inside a 16-row block
    const int slot_shift = gsh - 5;  // run index -> group index
    const int MC = 16 >> (7 - gsh);  // activation rows per pass

    const int64_t runs_per_row = K >> 5;
    const int64_t wpr = runs_per_row * BITS;  // packed words per row
    const int nspans = (int)((runs_per_row + 3) >> 2);
    const bool a_slot_ok = (lr / MC) == (lg >> slot_shift);

    constexpr uint32_t kOne = (BITS == 8) ? 0x3F803F80u : 0x43004300u;  // 1.0 or 128.0
    const bf16x8_t ones = as_bf16x8(kOne, kOne, kOne, kOne);

    f32x4_t acc[RB][NMC];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int c = 0; c < NMC; ++c) acc[rb][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // Word offsets of this lane's rows (clamped in range); packed weights are
    // limited to 2^32 words per matrix by the host, so offsets are 32-bit.
    uint32_t row_off[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int64_t row = row0 + rb * 16 + lr;
        row_off[rb] = (uint32_t)((row < R ? row : R - 1) * wpr);
    }
    const uint32_t last_run = (uint32_t)runs_per_row - 1;

    auto load = [&](int s, Stage<BITS, RB>& st) {
        const uint32_t run = (uint32_t)s * 4u + (uint32_t)lg;
        const uint32_t runc = run < last_run ? run : last_run;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            load_run_stream<BITS>(wq + (row_off[rb] + runc * BITS), st.cw[rb]);
            if constexpr (!SLDS) {
                const int64_t row = row0 + rb * 16 + lr;
                const int64_t gi = (row < R ? row : R - 1) * G + (runc >> slot_shift);
                st.sc[rb] = load_raw<SDT>(scales, gi);
                st.bi[rb] = load_raw<SDT>(biases, gi);
            }
        }
    };

    // The first NS-1 stages of packed codes are requested before the LDS
    // staging below, so their latency overlaps it.  (A wave past the end of
    // its problem loads clamped rows and leaves after the barrier.)
    const int s0 = (KS == 1) ? 0 : wave;
    Stage<BITS, RB> st[NS];
    if constexpr (SLDS) {
#pragma unroll
        for (int i = 0; i < NS - 1; ++i) {
            load(s0 + i * KS, st[i]);
            __builtin_amdgcn_sched_barrier(0);  // stage 0 must be the oldest load
        }
    }

    // LDS: 64 zero bytes (the A operand of inactive lanes, and a zero group
    // sum), x [M][K] bf16, the group sums X [M][G] fp32, then the block's
    // (scale, bias) pairs [kRowsPerBlock][G].
    uint16_t* xzero = lds;
    uint16_t* xs = lds + 32;
    const uint32_t xsum_f = (uint32_t)((64 + (((int64_t)M * K * 2 + 15) & ~15ll)) >> 2);
    float* xsum = (float*)lds + xsum_f;
    sbp_t* sbs = (sbp_t*)(xsum + (((int64_t)M * G + 3) & ~3ll));
    if constexpr (SLDS) {
        if (threadIdx.x < 4) *(u32x4_t*)&xzero[threadIdx.x * 8] = u32x4_t{0u, 0u, 0u, 0u};
        // Stage x[0..M) as bf16: 8 elements per thread per step.  With the
        // hi/lo split, rows M/2.. are the lo parts of rows 0..M/2-1.
        const int64_t n8 = (int64_t)M * K / 8;
        const int64_t half8 = args.xsplit ? n8 / 2 : n8;
        for (int64_t e = threadIdx.x; e < n8; e += kBlock) {
            uint32_t d[4];
            if (x_dt == RQ_BF16) {
                const uint4 v = ((const uint4*)x)[e];
                d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
            } else {
                const bool lo = e >= half8;
                const int64_t es = lo ? e - half8 : e;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float a = load_dt(x, x_dt, es * 8 + 2 * q);
                    const float b = load_dt(x, x_dt, es * 8 + 2 * q + 1);
                    d[q] = lo ? pair_lo(a, b) : pack_bf16x2(a, b);
                }
            }
            uint32_t pr[4];  // stored as pairs (x_i, x_{i+4}): the order of the code pairs
            reorder_pairs(d, pr);
            *(u32x4_t*)&xs[e * 8] = u32x4_t{pr[0], pr[1], pr[2], pr[3]};
            // Group sums of the bf16 values the MFMAs see.  A group is
            // gs/8 consecutive e, i.e. consecutive lanes of one wave (K and
            // the loop stride are multiples of gs/8), all active together.
            float sum = 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                sum += __uint_as_float(d[q] << 16) + __uint_as_float(d[q] & 0xffff0000u);
            for (int w = 1; w < (1 << (gsh - 3)); w <<= 1) sum += __shfl_xor(sum, w, 64);
            if ((e & ((1 << (gsh - 3)) - 1)) == 0) xsum[e >> (gsh - 3)] = sum;
        }
        // Stage the block's (scale, bias) pairs; rows past R are zero pairs.
        // With 16-bit scales, 16-byte aligned arrays and G % 8 == 0, eight
        // pairs per thread per step (two 128-bit loads, two 128-bit LDS
        // stores); otherwise one pair per step.
        const int64_t nsb = (int64_t)kRowsPerBlock * G;
        if (SDT != RQ_F32 && args.sb_vec && (G & 7) == 0) {
            for (int64_t e8 = threadIdx.x; e8 < nsb / 8; e8 += kBlock) {
                const int64_t e = e8 * 8;
                const int64_t rl = e / G, g = e - rl * G;
                const int64_t row = blk_row0 + rl;
                u32x4_t sv = {0u, 0u, 0u, 0u}, bv = {0u, 0u, 0u, 0u};
                if (row < R) {
                    sv = *(const u32x4_t*)((const uint16_t*)scales + row * G + g);
                    bv = *(const u32x4_t*)((const uint16_t*)biases + row * G + g);
                }
                uint32_t o[8];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    o[2 * q] = (sv[q] & 0xffffu) | (bv[q] << 16);
                    o[2 * q + 1] = (sv[q] >> 16) | (bv[q] & 0xffff0000u);
                }
                u32x4_t* dst = (u32x4_t*)&sbs[e];
                dst[0] = u32x4_t{o[0], o[1], o[2], o[3]};
                dst[1] = u32x4_t{o[4], o[5], o[6], o[7]};
            }
        } else
        for (int64_t e = threadIdx.x; e < nsb; e += kBlock) {
            const int64_t rl = e / G, g = e - rl * G;
            const int64_t row = blk_row0 + rl;
            sbp_t v;
            if constexpr (SDT == RQ_F32) {
                v = row < R ? make_uint2(((const uint32_t*)scales)[row * G + g],
                                         ((const uint32_t*)biases)[row * G + g])
                            : make_uint2(0u, 0u);
            } else {
                v = row < R ? (uint32_t)((const uint16_t*)scales)[row * G + g] |
                                  ((uint32_t)((const uint16_t*)biases)[row * G + g] << 16)
                            : 0u;
            }
            sbs[e] = v;
        }
        __syncthreads();
    }
    if (row0 >= R) return;  // a wave past the end of its problem (after the barrier)

    const PairConsts kc = pair_consts();
    // Per-lane constants of the staged path: LDS byte address of this lane's
    // activation row for each pass (or of the zero line when the lane's A row
    // is inactive), its row's (scale, bias) base and whether its rows exist.
    // (Indices are in 16-bit units of the dynamic LDS array: the zero line
    // is lds[0..32), x row m starts at lds[32 + m*K].)
    uint32_t a_idx[NMC], a_step[NMC];
#pragma unroll
    for (int c = 0; c < NMC; ++c) {
        const int m = c * MC + (lr % MC);
        const bool act = a_slot_ok && m < M;
        a_idx[c] = act ? (uint32_t)(32 + (int64_t)m * K + lg * 32) : 0u;
        a_step[c] = act ? 4u * 32u : 0u;  // elements per span (4 runs)
    }
    // LDS float index of the group sum for D row 4*lg+i in pass c (0, a zero,
    // when that row carries no activation row), and its step per span.
    constexpr int kMI = SLDS ? MI : 1;
    uint32_t g_idx[NMC][kMI], g_step[NMC][kMI];
    const int slots_per_span = 4 >> slot_shift;
#pragma unroll
    for (int c = 0; c < NMC; ++c)
#pragma unroll
        for (int i = 0; i < kMI; ++i) {
            const int m = c * MC + ((4 * lg + i) % MC);
            const bool act = m < M;
            g_idx[c][i] = act ? xsum_f + (uint32_t)(m * G + (lg >> slot_shift)) : 0u;
            g_step[c][i] = act ? (uint32_t)slots_per_span : 0u;
        }
    uint32_t sb_base[RB];
    bool row_ok[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int64_t row = row0 + rb * 16 + lr;
        row_ok[rb] = row < R;
        sb_base[rb] = (uint32_t)((row < R ? row - blk_row0 : 0) * G);
    }

    auto compute = [&](int s, const Stage<BITS, RB>& st) {
        const uint32_t run = (uint32_t)s * 4u + (uint32_t)lg;
        const bool run_ok = run <= last_run;
        bf16x8_t a[NMC][4];
        f32x4_t o[NMC];
        float xg[NMC][kMI];
#pragma unroll
        for (int c = 0; c < NMC; ++c) {
            const int m = c * MC + (lr % MC);
            uint32_t xd[16];
            if constexpr (SLDS) {
                // Branch-free: inactive lanes and runs past K read the zero
                // line (a zero scale alone would not cancel Inf/NaN garbage).
                const uint32_t ai = run_ok ? a_idx[c] + (uint32_t)s * a_step[c] : 0u;
                const u32x4_t* src = (const u32x4_t*)&lds[ai];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const u32x4_t v = src[q];
                    xd[4 * q] = v[0]; xd[4 * q + 1] = v[1]; xd[4 * q + 2] = v[2]; xd[4 * q + 3] = v[3];
                }
#pragma unroll
                for (int i = 0; i < kMI; ++i) {
                    const uint32_t gi = run_ok ? g_idx[c][i] + (uint32_t)s * g_step[c][i] : 0u;
                    xg[c][i] = ((const float*)lds)[gi];
                }
            } else if (a_slot_ok && run_ok && m < M) {
                const int msrc = args.xsplit ? M / 2 : M;  // rows msrc.. are lo parts
                const int64_t off = (int64_t)(m < msrc ? m : m - msrc) * K + run * 32;
                if (x_dt == RQ_BF16) load_x_run_bf16<RQ_BF16>(x, off, xd);
                else if (m >= msrc) load_x_run_lo(x, x_dt, off, xd);
                else if (x_dt == RQ_F32) load_x_run_bf16<RQ_F32>(x, off, xd);
                else load_x_run_bf16<RQ_F16>(x, off, xd);
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) xd[i] = 0u;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (SLDS) {  // staged already in pair order
                    a[c][j] = as_bf16x8(xd[4 * j], xd[4 * j + 1], xd[4 * j + 2], xd[4 * j + 3]);
                } else {
                    uint32_t pr[4];
                    reorder_pairs(&xd[4 * j], pr);
                    a[c][j] = as_bf16x8(pr[0], pr[1], pr[2], pr[3]);
                }
            }
            if constexpr (!SLDS) {
                o[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[c][j], ones, o[c], 0, 0, 0);
            }
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            bf16x8_t bop[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t pr[4];
                codes_to_bf16_pairs<BITS>(st.cw[rb], j, pr, kc);
                bop[j] = as_bf16x8(pr[0], pr[1], pr[2], pr[3]);
            }
            float sc, bi;
            if constexpr (SLDS) {
                // Rows past R have zero pairs in LDS; runs past K have zero
                // activations and group sums, so their (clamped, finite)
                // scale multiplies zeros.
                const uint32_t runc = run_ok ? run : last_run;
                const sbp_t v = sbs[sb_base[rb] + (runc >> slot_shift)];
                if constexpr (SDT == RQ_F32) {
                    sc = __uint_as_float(v.x);
                    bi = __uint_as_float(v.y);
                } else {
                    sc = raw_to_f32<SDT>(v & 0xffffu);
                    bi = raw_to_f32<SDT>(v >> 16);
                }
            } else {
                const bool ok = run_ok && row_ok[rb];
                sc = ok ? raw_to_f32<SDT>(st.sc[rb]) : 0.f;
                bi = ok ? raw_to_f32<SDT>(st.bi[rb]) : 0.f;
            }
            // coefficient of the group sum (LDS path) or of O = 128 * sum
            const float cb = (BITS == 8) ? bi
                           : (SLDS ? fmaf(sc, -128.f, bi) : (bi * 0.0078125f - sc));
#pragma unroll
            for (int c = 0; c < NMC; ++c) {
                f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[c][j], bop[j], d, 0, 0, 0);
                if constexpr (SLDS) {
#pragma unroll
                    for (int i = 0; i < kMI; ++i)
                        acc[rb][c][i] = fmaf(sc, d[i], fmaf(cb, xg[c][i], acc[rb][c][i]));
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[rb][c][i] = fmaf(sc, d[i], fmaf(cb, o[c][i], acc[rb][c][i]));
                }
            }
        }
    };

    if constexpr (SLDS) {
        // Rolling pipeline: span s+(NS-1)*KS is loaded while span s is computed.
        for (int s = s0; s < nspans; s += NS * KS) {
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                load(s + (i + NS - 1) * KS, st[(i + NS - 1) % NS]);
                compute(s + i * KS, st[i]);
                // keep the loads in issue order: the memory counter retires in
                // order, so a stage loaded late would make its compute drain
                // every younger load
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else {
        // Batches of NS spans: all loads first, then consume in order.
        for (int s = s0; s < nspans; s += NS * KS) {
#pragma unroll
            for (int i = 0; i < NS; ++i) load(s + i * KS, st[i]);
#pragma unroll
            for (int i = 0; i < NS; ++i) compute(s + i * KS, st[i]);
        }
    }

    if constexpr (KS > 1) {
        __shared__ float red[KS][RB][NMC][4][64];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int c = 0; c < NMC; ++c)
#pragma unroll
                for (int i = 0; i < 4; ++i) red[wave][rb][c][i][lane] = acc[rb][c][i];
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int c = 0; c < NMC; ++c)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float v = red[0][rb][c][i][lane];
#pragma unroll
                    for (int w = 1; w < KS; ++w) v += red[w][rb][c][i][lane];
                    acc[rb][c][i] = v;
                }
    }

    // Slot combine: D row m' = slot*MC + mm lives in lane group (m'/4), so the
    // slots of one output meet with xor-shuffles across lane groups.
    const int slots = 16 / MC;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int64_t row = row0 + rb * 16 + lr;
        if (args.xsplit) {
            // M <= 4 rows, all in lane group 0's accumulator rows 0..M-1:
            // output row i is the hi row i plus the lo row i + M/2
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = acc[rb][0][i];
                if (slots == 4) v[i] += __shfl_xor(v[i], 16, 64);
                if (slots >= 2) v[i] += __shfl_xor(v[i], 32, 64);
            }
            if (lg == 0 && row < R) {
                store_dt(args.p[p].y, args.y_dt, row, v[0] + (M == 2 ? v[1] : v[2]));
                if (M == 4) store_dt(args.p[p].y, args.y_dt, R + row, v[1] + v[3]);
            }
            continue;
        }
#pragma unroll
        for (int c = 0; c < NMC; ++c) {
#pragma unroll
            for (int i = 0; i < (SLDS ? kMI : 4); ++i) {
                float v = acc[rb][c][i];
                if (slots == 4) v += __shfl_xor(v, 16, 64);
                if (slots >= 2) v += __shfl_xor(v, 32, 64);
                const int m = c * MC + 4 * lg + i;
                if (lg < MC / 4 && m < M && row < R)
                    store_dt(args.p[p].y, args.y_dt, (int64_t)m * R + row, v);
            }
        }
    }
}

template <int SDT, int NMC, int MI, int RB, int KS, bool XLDS>
hipError_t launch_one(const QmvArgs& a, int blocks, size_t lds, hipStream_t stream) {
    constexpr int NS = XLDS ? RQ_QMV_NS : RQ_QMV_BATCH;
    hipLaunchKernelGGL((qmv_kernel<RQ_BITS, SDT, NMC, MI, RB, KS, NS, XLDS>), dim3(blocks),
                       dim3(kBlock), lds, stream, a);
    return hipGetLastError();
}

template <int RB, int KS>
hipError_t launch_cfg(const QmvArgs& a, int sb_dt, int nmc, bool xlds, int blocks, size_t lds,
                      hipStream_t stream) {
    hipError_t e = hipErrorInvalidValue;
    // MI: accumulator rows that can carry activations (see the kernel)
    const int mi = a.m >= 3 ? 4 : a.m;
#define RQ_QMV_NMC(SD, XL)                                                                \
    switch (nmc * 8 + (nmc == 1 ? mi : 4)) {                                              \
        case 9: e = launch_one<SD, 1, 1, RB, KS, XL>(a, blocks, lds, stream); break;       \
        case 10: e = launch_one<SD, 1, 2, RB, KS, XL>(a, blocks, lds, stream); break;      \
        case 12: e = launch_one<SD, 1, 4, RB, KS, XL>(a, blocks, lds, stream); break;      \
        case 20: e = launch_one<SD, 2, 4, RB, KS, XL>(a, blocks, lds, stream); break;      \
        case 36: e = launch_one<SD, 4, 4, RB, KS, XL>(a, blocks, lds, stream); break;      \
        default: break;                                                                   \
    }
    RQ_DISPATCH_DT(sb_dt, SD, if (xlds) { RQ_QMV_NMC(SD, true) } else { RQ_QMV_NMC(SD, false) });
#undef RQ_QMV_NMC
    return e;
}


// ------------------------------------------------------------ streamed GEMV
//
// qmv_stream_*: the decode GEMV for the common layout -- 16-bit scales with
// 16-byte aligned arrays and K a multiple of 512 -- built around full cache
// lines and streamed (scale, bias) pairs:
//
//  * A "stage" is 256 codes of 16 weight rows.  Lane L takes the two
//    consecutive runs 2g, 2g+1 (g = L/16) of row L%16: 64 contiguous codes,
//    so one wave-load covers 16 rows x 128 B, whole cache lines (measured:
//    +18% streaming rate over 16 rows x 64 B per load).  Stage s+1 is in
//    flight while stage s is computed (s+3 at 32-code groups).
//  * Each lane group owns a different k-slice of the MFMA, so the 16 A rows
//    are split into 4 slots (A row m' carries x[m'%4] on lane group m'/4's
//    slice only): D row 4g+i sums exactly lane group g's codes, i.e. one
//    group (two at gs=32: the stage's two MFMA halves are kept apart), and
//    lane L's accumulator rows need only its own row's (scale, bias) and
//    the activation sums X of its own group(s).  This kernel takes m <= 4;
//    larger m runs the wide kernel below, whose MFMA rows are all
//    activation rows.
//  * Once per 64 groups a wave loads the (scale, bias) values of those
//    groups for its 16 rows (lane groups 0/2 take scales, 1/3 biases), one
//    window ahead, and parks them in its own LDS window (wave-private, no
//    barrier).
//  * Only x (pair-permuted bf16) and its sums X over 32-element (gs=32) or
//    64-element slices -- a lane group's k-slice never spans two groups and
//    at gs=128 covers half of one -- are staged per block, behind one
//    barrier.  acc += s * D + (b - 128 s) * X (8-bit: b * X).
//  * qmv_stream_table reads its problem from a device-side table (one entry
//    per block: problem << 16 | 64-row block of that problem), so one launch
//    covers any number of problems; blocks are ordered longest first by the
//    host.  qmv_stream_inline takes up to RQ_MAX_GROUPED problems in its
//    arguments.
constexpr int kZeroElems = 64;  // zero line at the start of LDS: 128 B (8 A fragments)
constexpr int kStreamSlotsMax = 4;  // largest m of the slotted streamed kernel; above: the wide one

#ifndef RQ_QMV_WIN_G
#define RQ_QMV_WIN_G 32
#endif
// Streamed GEMV, groups of 64 codes or more: stages per iteration, NS - 1 of
// them in flight.  Two (one stage ahead, 76 VGPRs at m = 1, 6 waves per
// SIMD) measured faster than four (98 VGPRs, 4 waves): the config-2 sweep
// 5.89 vs 5.67-5.71 TB/s, the head's single launch 17.6 vs 19.0-19.3 us;
// eight (7 ahead) was slower still (5.1 TB/s).
#ifndef RQ_QMV_STREAM_NS
#define RQ_QMV_STREAM_NS 2
#endif
// (scale, bias) windows: a window is RQ_QMV_WIN_G groups of a row (64 B of
// each array at 16-bit scales), loaded once for the IPW iterations that read
// it.  Loaded in 32-B parts one iteration apart, a 128-B line was often
// evicted from L2 in between and fetched again: an iteration takes about as
// long as the streamed codes need to turn the L2 over.  64 groups (whole
// lines) would remove the rest of the refetch at K >= 4096 but need 8 more
// VGPRs per lane, one wave per SIMD less at 4 bits.
template <int GSH, int WGV = RQ_QMV_WIN_G, int NSV = 4>
struct StreamWin {
    static constexpr int GPS = 256 >> GSH;             // groups per stage: 8, 4, 2
    static constexpr int GPI = NSV * GPS;              // groups per iteration (4 stages: 32, 16, 8)
    static constexpr int WG = WGV;                     // groups per window
    static constexpr int WW = WG * 2;                  // bytes per array per row per window
    static constexpr int IPW = WG / GPI;               // iterations per window: 2, 4, 8
    static constexpr int PB = GSH == 7 ? 8 : 16;       // load size: K % 512 == 0 keeps a row's
                                                       // array a multiple of PB bytes
    static constexpr int NP = WW / 2 / PB;             // loads per lane and window
    static constexpr int ROWB = 2 * WW + 16;           // LDS row stride (spreads the banks)
    static constexpr int WAVE_BYTES = 16 * ROWB;
    static_assert(IPW >= 1 && WG % GPI == 0, "a window holds whole iterations");
};

template <int N>
struct Words {
    uint32_t w[N];
};

// Pointers into global memory.  The problem descriptors of a table launch
// are loaded from memory, so without the address space the compiler emits
// FLAT loads, which also count as LDS operations: every wait for an LDS
// read would then wait for all code loads in flight.
#define RQ_GLOBAL __attribute__((address_space(1)))
typedef const RQ_GLOBAL uint32_t* gptr_u32;
typedef const RQ_GLOBAL uint16_t* gptr_u16;
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// 3-bit codes of a lane's 64-code slice (six words, LSB first) as bf16 pairs
// (c_p, c_{p+4}), p = 32h + 8j + i, i = 0..3 -- the pair order of the 4-bit
// path, so x is staged the same way.  One funnel shift puts c_p at bits 4..6
// of the low half and c_{p+4} (12 bits further) at bits 0..2 of the high
// half; one v_and_or_b32 with mask 0x00070070 and exponent bits 0x43004100
// then gives the exact bf16 values 8 + c_p (0x4100 | c << 4: unit 1/16 at
// 8.0) and 128 + c_{p+4}.  Low-half positions are the elements k % 8 < 4.
RQ_DEV PairConsts pair3_consts() {
    PairConsts c{0x00070070u, 0x43004100u};
    asm volatile("" : "+v"(c.mask), "+v"(c.magic));
    return c;
}
RQ_DEV void codes3_to_bf16_pairs(const uint32_t* w, int h, int j, uint32_t* out,
                                 const PairConsts& k) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int pos = 3 * (32 * h + 8 * j + i) - 4;  // bit of the slice at bit 0 of v
        uint32_t v;
        if (pos < 0) {
            v = w[0] << (-pos);
        } else {
            const int wi = pos >> 5, s = pos & 31;
            // the last word needs no funnel: c_{p+4} ends at bit s + 18 < 32 there
            v = s == 0 ? w[wi] : (wi < 5 ? __builtin_amdgcn_alignbit(w[wi + 1], w[wi], s) : w[wi] >> s);
        }
        out[i] = (v & k.mask) | k.magic;
    }
}

template <int BITS>
RQ_DEV void load_two_runs(gptr_u32 p, uint32_t* out) {
    // 2*BITS contiguous words; 16-byte aligned for even BITS, 8-byte for odd
    if constexpr ((BITS & 1) == 0) {
#pragma unroll
        for (int q = 0; q < BITS / 2; ++q) {
            const u32x4_t v = *((const RQ_GLOBAL u32x4_t*)p + q);
            out[4 * q] = v[0]; out[4 * q + 1] = v[1]; out[4 * q + 2] = v[2]; out[4 * q + 3] = v[3];
        }
    } else {
#pragma unroll
        for (int q = 0; q < BITS; ++q) {
            const u32x2_t v = *((const RQ_GLOBAL u32x2_t*)p + q);
            out[2 * q] = v[0]; out[2 * q + 1] = v[1];
        }
    }
}

// One (scale, bias) window load of a lane: NP loads of PB bytes of the row
// array `sbrow` (scales for lane groups 0/2, biases for 1/3) starting at
// group w*WG + part.  The window after the last one is never read: it loads
// `spare` instead (the activations: L2-resident, 16-byte aligned, >= 1 KB),
// so the load stays unconditional without fetching scale lines again.
template <int GSH, int WGV = RQ_QMV_WIN_G>
RQ_DEV Words<StreamWin<GSH, WGV>::WW / 8> load_sb_window(gptr_u16 sbrow, int part, int G, int w,
                                                          const void* spare) {
    typedef StreamWin<GSH, WGV> W;
    constexpr int GP = W::PB / 2;  // groups per load
    Words<W::WW / 8> v;
    const bool live = w * W::WG < G;
#pragma unroll
    for (int q = 0; q < W::NP; ++q) {
        int g = w * W::WG + part + q * GP;
        g = g < G - GP ? g : G - GP;  // past the row's end (G < 64): any valid data
        const gptr_u16 src = live ? sbrow + g : (gptr_u16)spare;
        if constexpr (W::PB == 16) {
            const u32x4_t a = *(const RQ_GLOBAL u32x4_t*)src;
            v.w[4 * q] = a[0]; v.w[4 * q + 1] = a[1]; v.w[4 * q + 2] = a[2]; v.w[4 * q + 3] = a[3];
        } else {
            const u32x2_t a = *(const RQ_GLOBAL u32x2_t*)src;
            v.w[2 * q] = a[0]; v.w[2 * q + 1] = a[1];
        }
    }
    return v;
}

// Eight consecutive activations as loaded (16 B of bf16/f16, 32 B of f32) and
// their conversion to four bf16-pair dwords in natural order.
struct XRaw {
    u32x4_t lo, hi;
};
RQ_DEV XRaw load_x8(const void* x, int x_dt, int64_t e) {  // e: index of the 8-element piece
    XRaw r;
    if (x_dt == RQ_F32) {
        const RQ_GLOBAL u32x4_t* p = (const RQ_GLOBAL u32x4_t*)x + 2 * e;
        r.lo = p[0];
        r.hi = p[1];
    } else {
        r.lo = ((const RQ_GLOBAL u32x4_t*)x)[e];  // r.hi unused
    }
    return r;
}
// Eight fp32 or f16 activations as the lo part of their split, natural order.
RQ_DEV void x8_to_bf16_lo(const XRaw& r, int x_dt, uint32_t* d) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float a, b;
        if (x_dt == RQ_F32) {
            const u32x4_t& v = q < 2 ? r.lo : r.hi;
            a = __uint_as_float(v[2 * (q & 1)]);
            b = __uint_as_float(v[2 * (q & 1) + 1]);
        } else {
            a = f16_bits_to_f32(r.lo[q] & 0xffffu);
            b = f16_bits_to_f32(r.lo[q] >> 16);
        }
        d[q] = pair_lo(a, b);
    }
}
RQ_DEV void x8_to_bf16(const XRaw& r, int x_dt, uint32_t* d) {
    if (x_dt == RQ_BF16) {
        d[0] = r.lo[0]; d[1] = r.lo[1]; d[2] = r.lo[2]; d[3] = r.lo[3];
    } else if (x_dt == RQ_F32) {
        d[0] = pack_bf16x2(__uint_as_float(r.lo[0]), __uint_as_float(r.lo[1]));
        d[1] = pack_bf16x2(__uint_as_float(r.lo[2]), __uint_as_float(r.lo[3]));
        d[2] = pack_bf16x2(__uint_as_float(r.hi[0]), __uint_as_float(r.hi[1]));
        d[3] = pack_bf16x2(__uint_as_float(r.hi[2]), __uint_as_float(r.hi[3]));
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            d[q] = pack_bf16x2(f16_bits_to_f32(r.lo[q] & 0xffffu), f16_bits_to_f32(r.lo[q] >> 16));
    }
}

template <int BITS, int SDT, int NMC, int MI, int GSH>
RQ_DEV void qmv_stream_body(const rq_problem& P, int lblock, int M, int x_dt, int y_dt, int xsplit) {
    static_assert(SDT != RQ_F32, "streamed scales are 16-bit");
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    // stages per iteration; NS-1 stages of codes in flight
    constexpr int NS = GSH >= 6 ? RQ_QMV_STREAM_NS : 4;
    typedef StreamWin<GSH, RQ_QMV_WIN_G, NS> W;
    typedef Words<W::WW / 2 / 4> win_t;  // a lane's half of one array's window row

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lg = lane >> 4, lr = lane & 15;
    const int64_t R = P.rows, K = P.cols;
    const int G = (int)(K >> GSH);
    const int nst = (int)(K >> 8);
    const int niter = (nst + NS - 1) / NS;
    const int64_t row0 = (int64_t)lblock * 64 + wave * 16;
    const int64_t rowc = (row0 + lr) < R ? (row0 + lr) : R - 1;
    const int64_t wpr = (K >> 5) * BITS;

    // ---- first loads: window 0, then codes of stages 0..NS-2
    const gptr_u16 sbrow = (gptr_u16)((lg & 1) ? P.biases : P.scales) + rowc * G;
    const int part = (lg >> 1) * (W::WG / 2);
    auto load_win = [&](int w) -> win_t { return load_sb_window<GSH>(sbrow, part, G, w, P.x); };
    const gptr_u32 wqr = (gptr_u32)P.w_q + rowc * wpr + lg * 2 * BITS;
    auto load_codes = [&](int st, uint32_t* words) {
        const int sc = st < nst ? st : nst - 1;
        load_two_runs<BITS>(wqr + sc * (8 * BITS), words);
    };
    win_t wv = load_win(0);
    uint32_t cw[NS][2 * BITS];
#pragma unroll
    for (int i = 0; i < NS - 1; ++i) {
        load_codes(i, cw[i]);
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- stage x [M][K] (bf16, pair order) and its group sums; zero line
    uint16_t* xs = lds + kZeroElems;
    constexpr int XSH = GSH < 6 ? GSH : 6;  // activation sums over 2^XSH elements
    const int GX = (int)(K >> XSH);
    const uint32_t xsum_f = (uint32_t)((2 * kZeroElems + (((int64_t)M * K * 2 + 15) & ~15ll)) >> 2);
    float* xsum = (float*)lds + xsum_f;
    // 3-bit: a second array of sums over the low-half positions (k % 8 < 4)
    constexpr int NSUM = BITS == 3 ? 2 : 1;
    const uint32_t xlo_d = (uint32_t)(((int64_t)M * GX + 3) & ~3ll);  // offset of that array
    uint8_t* win = (uint8_t*)(xsum + NSUM * xlo_d) + wave * W::WAVE_BYTES;
    if (threadIdx.x < kZeroElems / 8) *(u32x4_t*)&lds[threadIdx.x * 8] = u32x4_t{0u, 0u, 0u, 0u};
    {
        const void* __restrict__ x = P.x;
        const int64_t n8 = (int64_t)M * K / 8;
        const int64_t half8 = xsplit ? n8 / 2 : n8;  // rows M/2.. are the lo parts
        for (int64_t e = threadIdx.x; e < n8; e += kBlock) {
            uint32_t d[4];
            const bool lopart = e >= half8;
            const XRaw r = load_x8(x, x_dt, lopart ? e - half8 : e);
            if (lopart) x8_to_bf16_lo(r, x_dt, d);
            else x8_to_bf16(r, x_dt, d);
            uint32_t pr[4];
            reorder_pairs(d, pr);
            *(u32x4_t*)&xs[e * 8] = u32x4_t{pr[0], pr[1], pr[2], pr[3]};
            float sum = 0.f, lo = 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float v = __uint_as_float(d[q] << 16) + __uint_as_float(d[q] & 0xffff0000u);
                sum += v;
                if (q < 2) lo += v;
            }
#pragma unroll
            for (int w = 1; w < (1 << (XSH - 3)); w <<= 1) {
                sum += __shfl_xor(sum, w, 64);
                if constexpr (BITS == 3) lo += __shfl_xor(lo, w, 64);
            }
            if ((e & ((1 << (XSH - 3)) - 1)) == 0) {
                xsum[e >> (XSH - 3)] = sum;
                if constexpr (BITS == 3) xsum[xlo_d + (e >> (XSH - 3))] = lo;
            }
        }
    }
    __syncthreads();
    if (row0 >= R) return;  // no rows for this wave (after the barrier)

    // ---- per-lane constants
    const PairConsts kc = BITS == 3 ? pair3_consts() : pair_consts();
    // A: lane (lr, lg) supplies row m' = lr on lane group lg's k-slice; that
    // row carries x[c*4 + lr%4] when its slot lr/4 is lg.
    uint32_t a_idx[NMC], a_step[NMC];
#pragma unroll
    for (int c = 0; c < NMC; ++c) {
        const int m = c * 4 + (lr & 3);
        const bool act = (lr >> 2) == lg && m < M;
        a_idx[c] = act ? (uint32_t)(kZeroElems + (int64_t)m * K + lg * 64) : 0u;
        a_step[c] = act ? 256u : 0u;
    }
    // activation sums of this lane's k-slice for its D rows m = c*4 + i
    constexpr int GL = GSH == 5 ? 2 : 1;                 // groups per lane per stage
    const int glane = GSH == 5 ? 2 * lg : (GSH == 6 ? lg : (lg >> 1));
    const int xlane = GSH == 5 ? 2 * lg : lg;
    uint32_t g_idx[NMC][MI], g_step[NMC][MI];
#pragma unroll
    for (int c = 0; c < NMC; ++c)
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int m = c * 4 + i;
            const bool act = m < M;
            g_idx[c][i] = act ? xsum_f + (uint32_t)(m * GX + xlane) : 0u;
            g_step[c][i] = act ? (uint32_t)(256 >> XSH) : 0u;
        }
    uint8_t* win_w = win + lr * W::ROWB + (lg & 1) * W::WW + (lg >> 1) * (W::WW / 2);
    const uint8_t* win_r = win + lr * W::ROWB + glane * 2;

    f32x4_t acc[NMC];
#pragma unroll
    for (int c = 0; c < NMC; ++c) acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int it = 0; it < niter; ++it) {
        const int itw = it % W::IPW;
        if (itw == 0) {
            // this window of (scale, bias) values into LDS, the next one into registers
            *(win_t*)win_w = wv;  // read below by other lanes of this wave (LDS runs in order)
            __builtin_amdgcn_wave_barrier();
            wv = load_win(it / W::IPW + 1);
        }
#pragma unroll
        for (int t = 0; t < NS; ++t) {
            const int st = it * NS + t;
            load_codes(st + NS - 1, cw[(t + NS - 1) % NS]);
            if (st < nst) {
                // scales and biases of this lane's group(s) at this stage
                float sc[GL], cb[GL], cl[GL];
#pragma unroll
                for (int q = 0; q < GL; ++q) {
                    const int gw = itw * W::GPI + t * W::GPS + q;  // group within the window
                    const uint16_t sr = *(const uint16_t*)(win_r + gw * 2);
                    const uint16_t br = *(const uint16_t*)(win_r + W::WW + gw * 2);
                    sc[q] = raw_to_f32<SDT>(sr);
                    const float bi = raw_to_f32<SDT>(br);
                    cb[q] = (BITS == 8) ? bi : fmaf(sc[q], -128.f, bi);
                    cl[q] = 120.f * sc[q];  // 3-bit: low-half positions carry 8, not 128
                }
                f32x4_t d[NMC][2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    bf16x8_t bop[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        uint32_t pr[4];
                        if constexpr (BITS == 3) codes3_to_bf16_pairs(cw[t], h, j, pr, kc);
                        else codes_to_bf16_pairs<BITS>(cw[t] + h * BITS, j, pr, kc);
                        bop[j] = as_bf16x8(pr[0], pr[1], pr[2], pr[3]);
                    }
#pragma unroll
                    for (int c = 0; c < NMC; ++c) {
                        const u32x4_t* src =
                            (const u32x4_t*)&lds[a_idx[c] + (uint32_t)st * a_step[c] + h * 32];
                        d[c][h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const u32x4_t v = src[j];
                            d[c][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                as_bf16x8(v[0], v[1], v[2], v[3]), bop[j], d[c][h], 0, 0, 0);
                        }
                    }
                }
#pragma unroll
                for (int c = 0; c < NMC; ++c)
#pragma unroll
                    for (int i = 0; i < MI; ++i) {
                        const float* xg = (const float*)lds + g_idx[c][i] + (uint32_t)st * g_step[c][i];
                        if constexpr (BITS == 3) {
                            const float* xl = xg + xlo_d;
#pragma unroll
                            for (int q = 0; q < GL; ++q)
                                acc[c][i] = fmaf(cl[q], xl[q], acc[c][i]);
                        }
                        if constexpr (GL == 2) {
                            acc[c][i] = fmaf(sc[0], d[c][0][i], fmaf(cb[0], xg[0], acc[c][i]));
                            acc[c][i] = fmaf(sc[1], d[c][1][i], fmaf(cb[1], xg[1], acc[c][i]));
                        } else {
                            acc[c][i] = fmaf(sc[0], d[c][0][i] + d[c][1][i],
                                             fmaf(cb[0], xg[0], acc[c][i]));
                        }
                    }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // sum the four slots (lane groups), then lane group 0 stores rows < R
    const int64_t row = row0 + lr;
    if (xsplit) {  // M = 2 or 4 rows: output row i is hi row i plus lo row i + M/2
        float v[MI];
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            v[i] = acc[0][i];
            v[i] += __shfl_xor(v[i], 16, 64);
            v[i] += __shfl_xor(v[i], 32, 64);
        }
        if (lg == 0 && row < R) {
            if constexpr (MI == 2) {
                store_dt(P.y, y_dt, row, v[0] + v[1]);
            } else if constexpr (MI == 4) {
                store_dt(P.y, y_dt, row, v[0] + (M == 2 ? v[1] : v[2]));
                if (M == 4) store_dt(P.y, y_dt, R + row, v[1] + v[3]);
            }
        }
        return;
    }
#pragma unroll
    for (int c = 0; c < NMC; ++c)
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            float v = acc[c][i];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            const int m = c * 4 + i;
            if (lg == 0 && m < M && row < R) store_dt(P.y, y_dt, (int64_t)m * R + row, v);
        }
}

#ifndef RQ_QMV_STREAM_WPE
#define RQ_QMV_STREAM_WPE 0  // >0: occupancy (waves per SIMD) requested for the streamed GEMV
#endif
#if RQ_QMV_STREAM_WPE > 0
#define RQ_STREAM_OCC __attribute__((amdgpu_waves_per_eu(RQ_QMV_STREAM_WPE)))
#else
#define RQ_STREAM_OCC
#endif

template <int BITS, int SDT, int NMC, int MI, int GSH>
__global__ __launch_bounds__(kBlock) RQ_STREAM_OCC void qmv_stream_inline(const QmvArgs args) {
    const int bid = blockIdx.x;
    int lo = 0, hi = args.n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (args.block_start[mid] <= bid) lo = mid; else hi = mid - 1;
    }
    qmv_stream_body<BITS, SDT, NMC, MI, GSH>(args.p[lo], bid - args.block_start[lo], args.m,
                                             args.x_dt, args.y_dt, args.xsplit);
}

template <int BITS, int SDT, int NMC, int MI, int GSH>
__global__ __launch_bounds__(kBlock) RQ_STREAM_OCC void qmv_stream_table(const rq::QmvTable a) {
    const uint32_t e = a.blocks[blockIdx.x];
    const rq_problem P = a.descs[e >> 16];
    qmv_stream_body<BITS, SDT, NMC, MI, GSH>(P, (int)(e & 0xffffu), a.m, a.x_dt, a.y_dt, a.xsplit);
}

// ------------------------------------------------------------ split GEMV
//
// qmv_split: the decode GEMV of launches too small to fill the GPU with rows
// (one projection, or the few independent projections of one step of a
// layer), where a launch costs its memory round trips rather than its bytes.
// m <= 4 activation rows run in one pass of the slotted MFMA rows, 4 < m <= 8
// in two passes (NMC) that share each stage's code conversion.
//
//  * A block is one 16-row tile; its KS waves split K into contiguous slices
//    of NSW stages (a stage is 256 codes of the 16 rows, laid out as in the
//    streamed GEMV: lane L holds the 64 codes 64(L/16).. of row L%16).
//  * Every global load of a wave is issued before any is waited for: its
//    slice of x (first, so that it can be staged while codes still arrive),
//    the (scale, bias) values of its slice (lane groups 0/2 scales, 1/3
//    biases, half a row each) and the codes of all its stages.  A wave
//    stages x (pair-permuted bf16, plus activation sums) and its (scale,
//    bias) values in a wave-private LDS region, so no barrier precedes the
//    MFMAs; the arithmetic per stage is the streamed GEMV's.
//  * The slices' per-row sums meet behind the block's only barrier; wave 0
//    adds them in wave order (deterministic) and stores y.
#ifndef RQ_SPLIT_WAVES
#define RQ_SPLIT_WAVES 16  // most waves (K slices) per block
#endif
constexpr int kSplitMaxWaves = RQ_SPLIT_WAVES;
constexpr int kSplitBlock = 64 * kSplitMaxWaves;

template <int GSH>
struct SplitSB {
    static constexpr int SB1 = (256 >> GSH) * 2;  // bytes of one array per row and stage
};

// stages per wave: the fewest (a power of two) that need at most
// kSplitMaxWaves waves; 0 if that exceeds 4 (not covered: at 16 waves per
// block a wave may hold 128 VGPRs, and 8 stages of codes need more)
__host__ __device__ inline int split_nsw(int64_t cols) {
    const int64_t nst = cols >> 8;
    for (int nsw = 1; nsw <= 4; nsw *= 2)
        if (nst <= (int64_t)nsw * kSplitMaxWaves) return nsw;
    return 0;
}
// Arrays of activation sums staged in LDS: two for 3-bit codes (all and
// low-half positions), one for m <= 2; 4- and 8-bit codes at m >= 3 take the
// sums from a constant-B MFMA on the same A fragments instead (measured per
// launch: [2048, 8192] at m = 8 13.71 -> 12.10 us, [2048, 2048] 7.30 ->
// 6.61; at m <= 2 the extra MFMAs cost more than the few staged sums).
__host__ __device__ constexpr int split_nsum(int bits, int m) {
    return bits == 3 ? 2 : (m <= 2 ? 1 : 0);
}
__host__ __device__ inline int split_wave_bytes(int m, int nsw, int gsh, int bits) {
    const int xsh = gsh < 6 ? gsh : 6;
    const int sbb = nsw * ((256 >> gsh) * 2);
    return 128 + m * nsw * 512 + split_nsum(bits, m) * m * ((nsw * 256) >> xsh) * 4 +
           16 * (2 * sbb + 16);
}

template <int BITS, int SDT, int NMC, int MI, int GSH, int NSW>
__global__ __launch_bounds__(kSplitBlock) void qmv_split(const QmvArgs args) {
    static_assert(SDT != RQ_F32, "split GEMV scales are 16-bit");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];
    constexpr int XSH = GSH < 6 ? GSH : 6;
    // activation sums from a constant-B MFMA (m >= 3: the passes of codes 12
    // and 20), else staged in LDS
    constexpr bool XMF = BITS != 3 && !(NMC == 1 && MI <= 2);
    constexpr int NSUM = split_nsum(BITS, NMC == 1 && MI <= 2 ? MI : 4);
    constexpr int KW = NSW * 256;                 // codes per row in a wave's slice
    constexpr int SBB = NSW * SplitSB<GSH>::SB1;  // bytes per row and array in a slice
    constexpr int SBH = SBB / 2;                  // bytes of it one lane loads
    // load width: at most 16 B and never across a stage, so that a short last
    // slice loads exactly its own stages
    constexpr int SBW = SBH < SplitSB<GSH>::SB1 ? SBH : (SplitSB<GSH>::SB1 < 16 ? SplitSB<GSH>::SB1 : 16);
    constexpr int SBN = SBH / SBW;                // loads per lane
    constexpr int ROWB = 2 * SBB + 16;
    constexpr int MR = NMC == 1 ? MI : 4 * NMC;   // activation rows at most
    constexpr int XP = (MR * KW / 8 + 63) / 64;   // 8-element x pieces per lane (upper bound)

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lg = lane >> 4, lr = lane & 15;
    const int bid = blockIdx.x;
    int lo = 0, hi = args.n - 1;  // last problem whose first block <= bid
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (args.block_start[mid] <= bid) lo = mid; else hi = mid - 1;
    }
    const rq_problem& P = args.p[lo];
    const int M = args.m, x_dt = args.x_dt;
    const int64_t R = P.rows, K = P.cols;
    const int nst = (int)(K >> 8);
    const int st0 = wave * NSW;                                // first stage of this wave
    const int nv = nst - st0 < NSW ? nst - st0 : NSW;          // its stages (>= 1)
    const int64_t row0 = (int64_t)(bid - args.block_start[lo]) * 16;
    const int64_t rowc = (row0 + lr) < R ? (row0 + lr) : R - 1;
    const int64_t wpr = (K >> 5) * BITS;

    // wave-private LDS: zero line | x slice [M][KW] | sums (NSUM arrays) | (scale, bias) rows
    const int wbytes = split_wave_bytes(M, NSW, GSH, BITS);
    uint8_t* wl = lds8 + wave * wbytes;
    uint16_t* xs = (uint16_t*)(wl + 128);
    float* xsum = (float*)(wl + 128 + M * KW * 2);
    const int gxw = KW >> XSH;  // sums per activation row in the slice
    uint8_t* sbl = (uint8_t*)(xsum + NSUM * M * gxw);

    // ---- issue every load: x slice, (scale, bias) values, codes
    const int n8 = M * nv * 32;  // 8-element x pieces of the slice
    const int msrc = args.xsplit ? M / 2 : M;  // rows msrc.. are the lo parts of rows 0..
    XRaw xr[XP];
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int e = lane + 64 * i;
        if (e < n8) {
            const int m = e / (nv * 32), kk = (e - m * nv * 32) * 8;
            const int ms = m < msrc ? m : m - msrc;
            xr[i] = load_x8(P.x, x_dt, ((int64_t)ms * K + (int64_t)st0 * 256 + kk) >> 3);
        }
    }
    const RQ_GLOBAL uint8_t* sbsrc =
        (const RQ_GLOBAL uint8_t*)((lg & 1) ? P.biases : P.scales) +
        (rowc * (K >> GSH)) * 2 + (int64_t)st0 * SplitSB<GSH>::SB1;
    uint32_t sbv[(SBH + 3) / 4];
#pragma unroll
    for (int q = 0; q < SBN; ++q) {
        // bytes past a short last slice are never read: load the slice start instead
        const int off = (lg >> 1) * SBH + q * SBW;
        const int so = off < nv * SplitSB<GSH>::SB1 ? off : 0;
        if constexpr (SBW == 16) {
            const u32x4_t v = *(const RQ_GLOBAL u32x4_t*)(sbsrc + so);
            sbv[4 * q] = v[0]; sbv[4 * q + 1] = v[1]; sbv[4 * q + 2] = v[2]; sbv[4 * q + 3] = v[3];
        } else if constexpr (SBW == 8) {
            const u32x2_t v = *(const RQ_GLOBAL u32x2_t*)(sbsrc + so);
            sbv[2 * q] = v[0]; sbv[2 * q + 1] = v[1];
        } else if constexpr (SBW == 4) {
            sbv[q] = *(const RQ_GLOBAL uint32_t*)(sbsrc + so);
        } else {
            sbv[0] = *(const RQ_GLOBAL uint16_t*)(sbsrc + so);
        }
    }
    const gptr_u32 wqr = (gptr_u32)P.w_q + rowc * wpr + lg * 2 * BITS;
    uint32_t cw[NSW][2 * BITS];
#pragma unroll
    for (int t = 0; t < NSW; ++t) {
        const int sc = st0 + (t < nv ? t : 0);
        load_two_runs<BITS>(wqr + sc * (8 * BITS), cw[t]);
    }

    // ---- stage x and its sums (waits for x only: it was requested first)
    if (lane < 8) *(u32x4_t*)(wl + lane * 16) = u32x4_t{0u, 0u, 0u, 0u};
    float* xlo = xsum + M * gxw;  // 3-bit: sums over the low-half positions
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int e = lane + 64 * i;
        if (e < n8) {
            const int m = e / (nv * 32), kk = (e - m * nv * 32) * 8;
            uint32_t d[4];
            if (m >= msrc) x8_to_bf16_lo(xr[i], x_dt, d);
            else x8_to_bf16(xr[i], x_dt, d);
            uint32_t pr[4];
            reorder_pairs(d, pr);
            *(u32x4_t*)&xs[m * KW + kk] = u32x4_t{pr[0], pr[1], pr[2], pr[3]};
            if constexpr (!XMF) {
                float sum = 0.f, lo4 = 0.f;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float v = __uint_as_float(d[q] << 16) + __uint_as_float(d[q] & 0xffff0000u);
                    sum += v;
                    if (q < 2) lo4 += v;
                }
                // a sum covers 2^(XSH-3) consecutive pieces = consecutive lanes
#pragma unroll
                for (int w = 1; w < (1 << (XSH - 3)); w <<= 1) {
                    sum += __shfl_xor(sum, w, 64);
                    if constexpr (BITS == 3) lo4 += __shfl_xor(lo4, w, 64);
                }
                if ((e & ((1 << (XSH - 3)) - 1)) == 0) {
                    const int si = m * gxw + (kk >> XSH);
                    xsum[si] = sum;
                    if constexpr (BITS == 3) xlo[si] = lo4;
                }
            }
        }
    }
    {   // (scale, bias) values of the slice: row lr, array lg&1, half lg>>1
        uint8_t* dst = sbl + lr * ROWB + (lg & 1) * SBB + (lg >> 1) * SBH;
#pragma unroll
        for (int q = 0; q < SBN; ++q) {
            if constexpr (SBW == 16)
                *(u32x4_t*)(dst + 16 * q) = u32x4_t{sbv[4 * q], sbv[4 * q + 1], sbv[4 * q + 2], sbv[4 * q + 3]};
            else if constexpr (SBW == 8)
                *(u32x2_t*)(dst + 8 * q) = u32x2_t{sbv[2 * q], sbv[2 * q + 1]};
            else if constexpr (SBW == 4)
                *(uint32_t*)(dst + 4 * q) = sbv[q];
            else
                *(uint16_t*)dst = (uint16_t)sbv[0];
        }
    }
    __builtin_amdgcn_wave_barrier();  // LDS writes above are read by other lanes of this wave

    // ---- per-lane constants (as in the streamed GEMV, on the slice); pass c
    // carries activation rows 4c .. 4c+3
    const PairConsts kc = BITS == 3 ? pair3_consts() : pair_consts();
    uint32_t a_base[NMC], a_step[NMC];
#pragma unroll
    for (int c = 0; c < NMC; ++c) {
        const int m_a = 4 * c + (lr & 3);
        const bool a_act = (lr >> 2) == lg && m_a < M;
        a_base[c] = a_act ? (uint32_t)(64 + m_a * KW + lg * 64) : 0u;  // in 16-bit units
        a_step[c] = a_act ? 256u : 0u;
    }
    constexpr int GL = GSH == 5 ? 2 : 1;
    const int glane = GSH == 5 ? 2 * lg : (GSH == 6 ? lg : (lg >> 1));
    const int xlane = GSH == 5 ? 2 * lg : lg;
    const uint32_t xsum_f = (uint32_t)((128 + M * KW * 2) >> 2);  // float index of xsum in wl
    uint32_t g_idx[NMC][MI], g_step[NMC][MI];
#pragma unroll
    for (int c = 0; c < NMC; ++c)
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const bool act = 4 * c + i < M;
            g_idx[c][i] = act ? xsum_f + (uint32_t)((4 * c + i) * gxw + xlane) : 0u;
            g_step[c][i] = act ? (uint32_t)(256 >> XSH) : 0u;
        }
    const uint8_t* sb_r = sbl + lr * ROWB + glane * 2;

    f32x4_t acc[NMC];
#pragma unroll
    for (int c = 0; c < NMC; ++c) acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // XMF: the activation sums of a lane group's codes are the same A
    // fragments against bf16 1.0 (D rows as the product's: slot lg, row m)
    constexpr uint32_t kOne = 0x3F803F80u;
    const bf16x8_t ones = as_bf16x8(kOne, kOne, kOne, kOne);
    const uint16_t* wl16 = (const uint16_t*)wl;
    const float* wlf = (const float*)wl;
#pragma unroll
    for (int t = 0; t < NSW; ++t) {
        if (t < nv) {
            float sc[GL], cb[GL], cl[GL];
#pragma unroll
            for (int q = 0; q < GL; ++q) {
                const int gw = t * (256 >> GSH) + q;
                sc[q] = raw_to_f32<SDT>(*(const uint16_t*)(sb_r + gw * 2));
                const float bi = raw_to_f32<SDT>(*(const uint16_t*)(sb_r + SBB + gw * 2));
                cb[q] = (BITS == 8) ? bi : fmaf(sc[q], -128.f, bi);
                cl[q] = 120.f * sc[q];
            }
            f32x4_t d[NMC][2], xm[NMC][GL];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                bf16x8_t bop[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint32_t pr[4];
                    if constexpr (BITS == 3) codes3_to_bf16_pairs(cw[t], h, j, pr, kc);
                    else codes_to_bf16_pairs<BITS>(cw[t] + h * BITS, j, pr, kc);
                    bop[j] = as_bf16x8(pr[0], pr[1], pr[2], pr[3]);
                }
#pragma unroll
                for (int c = 0; c < NMC; ++c) {
                    const u32x4_t* src =
                        (const u32x4_t*)&wl16[a_base[c] + (uint32_t)t * a_step[c] + h * 32];
                    constexpr int hx = GL == 2 ? 1 : 0;  // sums per run (gs 32) or per stage
                    d[c][h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
                    if (XMF && (GL == 2 || h == 0)) xm[c][h & hx] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const u32x4_t v = src[j];
                        const bf16x8_t a = as_bf16x8(v[0], v[1], v[2], v[3]);
                        d[c][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bop[j], d[c][h], 0, 0, 0);
                        if constexpr (XMF)
                            xm[c][h & hx] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                a, ones, xm[c][h & hx], 0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < NMC; ++c)
#pragma unroll
                for (int i = 0; i < MI; ++i) {
                    if constexpr (XMF) {
                        if constexpr (GL == 2) {
                            acc[c][i] = fmaf(sc[0], d[c][0][i], fmaf(cb[0], xm[c][0][i], acc[c][i]));
                            acc[c][i] = fmaf(sc[1], d[c][1][i], fmaf(cb[1], xm[c][GL - 1][i], acc[c][i]));
                        } else {
                            acc[c][i] = fmaf(sc[0], d[c][0][i] + d[c][1][i],
                                             fmaf(cb[0], xm[c][0][i], acc[c][i]));
                        }
                        continue;
                    }
                    const float* xg = wlf + g_idx[c][i] + (uint32_t)t * g_step[c][i];
                    if constexpr (BITS == 3) {
                        const float* xl = xg + M * gxw;
#pragma unroll
                        for (int q = 0; q < GL; ++q) acc[c][i] = fmaf(cl[q], xl[q], acc[c][i]);
                    }
                    if constexpr (GL == 2) {
                        acc[c][i] = fmaf(sc[0], d[c][0][i], fmaf(cb[0], xg[0], acc[c][i]));
                        acc[c][i] = fmaf(sc[1], d[c][1][i], fmaf(cb[1], xg[1], acc[c][i]));
                    } else {
                        acc[c][i] = fmaf(sc[0], d[c][0][i] + d[c][1][i], fmaf(cb[0], xg[0], acc[c][i]));
                    }
                }
        }
    }

    // ---- slots (lane groups) of a row meet by shuffles, slices in LDS
    float v[NMC][MI];
#pragma unroll
    for (int c = 0; c < NMC; ++c)
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            v[c][i] = acc[c][i];
            v[c][i] += __shfl_xor(v[c][i], 16, 64);
            v[c][i] += __shfl_xor(v[c][i], 32, 64);
        }
    const int ks = blockDim.x >> 6;
    float* red = (float*)(wl + 128);  // this wave's x slice is no longer read
    if (ks > 1) {
        __builtin_amdgcn_wave_barrier();
        if (lg == 0) {
#pragma unroll
            for (int c = 0; c < NMC; ++c)
#pragma unroll
                for (int i = 0; i < MI; ++i) red[(4 * c + i) * 16 + lr] = v[c][i];
        }
        __syncthreads();
        if (wave != 0) return;
        // lane group lg sums rows m = 4c + lg over the slices, in wave order
#pragma unroll
        for (int c = 0; c < NMC; ++c) {
            if (lg < MI) {
                float s = 0.f;
                for (int w = 0; w < ks; ++w)
                    s += ((const float*)(lds8 + w * wbytes + 128))[(4 * c + lg) * 16 + lr];
#pragma unroll
                for (int i = 0; i < MI; ++i)
                    if (i == lg) v[c][i] = s;
            }
        }
    }
    const int64_t row = row0 + lr;
    if (args.fold) {
        // rows 2r + p are the halves p of weight row r and activation rows
        // 2m + p the matching halves of x row m: lane (lg, lr) with lg and lr
        // even holds half 0 of output (m, r), lane + 17 half 1
        const int64_t rr = row >> 1;
#pragma unroll
        for (int c = 0; c < NMC; ++c) {
            float mine = 0.f;
#pragma unroll
            for (int i = 0; i < MI; ++i)
                if (i == lg) mine = v[c][i];
            const float other = __shfl(mine, (lane + 17) & 63, 64);
            const int m = 2 * c + (lg >> 1);
            if (((lg | lr) & 1) == 0 && lg < MI && 2 * m < M && rr < (R >> 1))
                store_dt(P.y, args.y_dt, (int64_t)m * (R >> 1) + rr, mine + other);
        }
        return;
    }
    if (args.xsplit) {
        // M = 2 or 4 rows in one pass, row i in lane group i: output row i is
        // hi row i plus lo row i + M/2, which lane group i + M/2 holds
        float mine = 0.f;
#pragma unroll
        for (int i = 0; i < MI; ++i)
            if (i == lg) mine = v[0][i];
        const float other = __shfl(mine, (lane + 16 * msrc) & 63, 64);
        if (lg < msrc && row < R) store_dt(P.y, args.y_dt, (int64_t)lg * R + row, mine + other);
        return;
    }
#pragma unroll
    for (int c = 0; c < NMC; ++c)
#pragma unroll
        for (int i = 0; i < MI; ++i)
            if (lg == i && 4 * c + i < M && row < R)
                store_dt(P.y, args.y_dt, (int64_t)(4 * c + i) * R + row, v[c][i]);
}

// ------------------------------------------------------------ wide GEMV
//
// qmv_wide_*: the decode GEMV for 4 < m <= 16 on the streamed layout (same
// stages, lane loads, (scale, bias) windows and launch forms as
// qmv_stream_*).  Lane group g of a wave holds the 64 codes (eight 8-code
// pieces) of 64-code unit g of a stage for its row.  After the loads
// arrive, pieces are exchanged between lane groups with v_permlane32_swap
// and v_permlane16_swap so that each MFMA's 32-element contraction holds
// codes of as few groups as the activation rows allow:
//
//  * m <= 8 (MP = 8, two slots): one swap per piece pair moves lane-group
//    bit 1 into the register index.  MFMA (P, v) then holds in lane group
//    2b + c piece 2v + b of unit 2P + c: A rows 0-7 carry x[m] on the units
//    2P pieces (lane groups 0 and 2), rows 8-15 on the 2P+1 pieces (lane
//    groups 1 and 3), zero elsewhere, so D rows 0-7 sum unit 2P and rows
//    8-15 unit 2P+1, and lane L's accumulator rows belong to one unit:
//    2P + (L/32).  Four MFMAs cover two units; the halves are summed across
//    lane groups g, g^2 at the end.
//  * m <= 16 (MP = 16, no slots): a full 4 x 4 transpose of (lane group,
//    piece) per run half (4 swaps per 4 words) makes MFMA (t, h) contract
//    exactly run 2t+h of the stage, with 16 activation rows.
//  * The activation sums over the same codes come from a second MFMA of the
//    same A fragment with a constant B (bf16 1.0), so only the pair-permuted
//    bf16 x is staged: per group, acc += s D + (b - 128 s) X (8-bit: b X).
//  * x lives in a two-slot LDS ring of 1024-column chunks (one iteration of
//    4 stages each), staged for the rows m < M; rows m >= M of the ring are
//    zero, and so is a 1024-column line that idle A lanes read.  Two
//    schedules:
//    - m <= 8 (MP = 8): the ring holds a pair of chunks (2048 columns); a row
//      of K <= 2048 is staged whole before the loop, a longer one restages
//      the next pair behind two barriers every two iterations.  This loop
//      takes ~116 VGPRs with one wait per stage for exactly its codes, and
//      (scale, bias) windows of 16 groups (32 at gs 32: one iteration) keep
//      the block at 40.2 KB of LDS: 4 waves per SIMD.
//    - m > 8 (MP = 16): K <= 2048 is staged whole up front; longer rows
//      stream chunks, the next chunk's loads issued at the start of an
//      iteration and written after its MFMAs, behind one barrier per
//      iteration.  Both loops live in one kernel.  At MP = 8 that form took
//      167 VGPRs (3 waves per SIMD), and the compiler's wait analysis,
//      merged over both loops, made the whole-x loop wait for code loads of
//      later stages (vmcnt(2)/vmcnt(4) where vmcnt(6) suffices, vmcnt(1) at
//      each window); the pair schedule measured +3 % on the config-2 sweep
//      at M = 8 (+5 % on its K = 2048 projections, equal on K = 8192).
// 4- and 8-bit codes: their pieces are whole words.
constexpr int kWideNS = 4;                // stages per iteration = per staged x chunk
constexpr int kWideKC = 256 * kWideNS;    // x columns per chunk
constexpr int kWideRow = kWideKC + 8;     // LDS row stride in elements (+16 B spreads the banks)
#ifndef RQ_QMV_WIDE_WIN_G
#define RQ_QMV_WIDE_WIN_G 16
#endif
template <int GSH>
constexpr int wide_win_g() {
    return StreamWin<GSH>::GPI > RQ_QMV_WIDE_WIN_G ? StreamWin<GSH>::GPI : RQ_QMV_WIDE_WIN_G;
}

// 4 x 4 transpose of (lane group, register): afterwards register j of lane
// group g holds what register g of lane group j held.
RQ_DEV void transpose_lane_groups(uint32_t& a, uint32_t& b, uint32_t& c, uint32_t& d) {
    const auto r0 = __builtin_amdgcn_permlane32_swap(a, c, false, false);  // rows 2,3 of a <-> rows 0,1 of c
    const auto r1 = __builtin_amdgcn_permlane32_swap(b, d, false, false);
    const auto r2 = __builtin_amdgcn_permlane16_swap(r0[0], r1[0], false, false);  // odd rows of a <-> even rows of b
    const auto r3 = __builtin_amdgcn_permlane16_swap(r0[1], r1[1], false, false);
    a = r2[0]; b = r2[1]; c = r3[0]; d = r3[1];
}

// codes_to_bf16_pairs<4> of two words at once: the shifted copies of both
// come from 64-bit shifts of the pair (3 shifts for 2 words instead of 6;
// bits shifted in from the other word fall outside the 0x000F000F mask).
#ifndef RQ_QMV_SHIFT64
#define RQ_QMV_SHIFT64 1
#endif
RQ_DEV void codes4_to_bf16_pairs_x2(uint32_t w0, uint32_t w1, uint32_t* o0, uint32_t* o1,
                                    const PairConsts& k) {
#if RQ_QMV_SHIFT64
    const uint64_t ww = ((uint64_t)w1 << 32) | w0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint64_t t = ww >> (4 * i);
        o0[i] = ((uint32_t)t & k.mask) | k.magic;
        o1[i] = ((uint32_t)(t >> 32) & k.mask) | k.magic;
    }
#else
    const uint32_t ws[2] = {w0, w1};
    codes_to_bf16_pairs<4>(ws, 0, o0, k);
    codes_to_bf16_pairs<4>(ws, 1, o1, k);
#endif
}

// Swap of lane groups 2, 3 of a with lane groups 0, 1 of b.
RQ_DEV void swap_lane_halves(uint32_t& a, uint32_t& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = r[0]; b = r[1];
}

template <int MP>
struct WideLds {
    static constexpr int ZERO = 2 * MP * kWideRow;   // zero line read by idle A lanes (MP = 8)
    static constexpr int DUMMY = ZERO + (MP == 8 ? kWideKC : 0);  // 16-B sink for idle stores
    static constexpr int X_ELEMS = DUMMY + 8;
};

// x schedule: at MP = 8 by pairs of chunks (restaged behind barriers); at
// MP = 16 whole when K <= 2048 and streamed chunk by chunk beyond.
template <int BITS, int SDT, int MP, int GSH, bool XF32>
RQ_DEV void qmv_wide_body(const rq_problem& P, int lblock, int M, int x_dt, int y_dt) {
    static_assert(BITS == 4 || BITS == 8, "wide GEMV: codes whose 8-code pieces are whole words");
    static_assert(SDT != RQ_F32, "streamed scales are 16-bit");
    static_assert(MP == 8 || MP == 16, "");
    constexpr bool XP = MP == 8;  // x by pairs of chunks, restaged behind barriers
    typedef StreamWin<GSH, XP ? wide_win_g<GSH>() : RQ_QMV_WIN_G> W;
    typedef WideLds<MP> L;
    __shared__ __attribute__((aligned(16))) uint16_t xring[L::X_ELEMS];
    __shared__ __attribute__((aligned(16))) uint8_t wins[kWaves * W::WAVE_BYTES];
    constexpr int NS = kWideNS;
    constexpr int PW = BITS / 4;                                       // words per 8-code piece
    constexpr int XQ = (MP * (kWideKC / 8) + kBlock - 1) / kBlock;     // x pieces per thread per chunk
    typedef Words<W::WW / 8> win_t;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lg = lane >> 4, lr = lane & 15;
    const int64_t R = P.rows, K = P.cols;
    const int G = (int)(K >> GSH);
    const int nst = (int)(K >> 8);
    const int niter = (nst + NS - 1) / NS;
    const int64_t row0 = (int64_t)lblock * 64 + wave * 16;
    const int64_t rowc = (row0 + lr) < R ? (row0 + lr) : R - 1;
    const int64_t wpr = (K >> 5) * BITS;

    // ---- first loads: window 0, then codes of stages 0..NS-2
    const gptr_u16 sbrow = (gptr_u16)((lg & 1) ? P.biases : P.scales) + rowc * G;
    const int part = (lg >> 1) * (W::WG / 2);
    win_t wv = load_sb_window<GSH, W::WG>(sbrow, part, G, 0, P.x);
    const gptr_u32 wqr = (gptr_u32)P.w_q + rowc * wpr + lg * 2 * BITS;
    auto load_codes = [&](int st, uint32_t* words) {
        const int sc = st < nst ? st : nst - 1;
        load_two_runs<BITS>(wqr + sc * (8 * BITS), words);
    };
    uint32_t cw[NS][2 * BITS];
#pragma unroll
    for (int i = 0; i < NS - 1; ++i) {
        load_codes(i, cw[i]);
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- x chunks: piece e of a chunk is row e / 128, columns 8 (e % 128) ..
    // Loads and stores of a chunk are unconditional (a chunk past the last
    // reloads the last, idle pieces go to a sink): the compiler's wait
    // analysis is path-insensitive, so loads left unconsumed on any path
    // around the loop made it wait at the loop head for every load issued
    // after them, the code pipeline included.  (x_dt is a template choice
    // between f32 and 16-bit here for the same reason.)
    const int npc = M * (kWideKC / 8);
    const int64_t k8 = K >> 3;
    auto load_chunk = [&](int c, XRaw* xr) {
        c = c < niter ? c : niter - 1;
#pragma unroll
        for (int q = 0; q < XQ; ++q) {
            const int e = threadIdx.x + q * kBlock;
            const int64_t col8 = (int64_t)c * (kWideKC / 8) + (e & 127);
            const bool ok = e < npc && col8 < k8;
            const int64_t i = ok ? (int64_t)(e >> 7) * k8 + col8 : 0;
            if constexpr (XF32) {
                const RQ_GLOBAL u32x4_t* src = (const RQ_GLOBAL u32x4_t*)P.x + 2 * i;
                xr[q].lo = src[0];
                xr[q].hi = src[1];
            } else {
                xr[q].lo = ((const RQ_GLOBAL u32x4_t*)P.x)[i];
            }
        }
    };
    auto store_chunk = [&](int slot, const XRaw* xr) {
#pragma unroll
        for (int q = 0; q < XQ; ++q) {
            const int e = threadIdx.x + q * kBlock;
            uint32_t d[4], pr[4];
            x8_to_bf16(xr[q], XF32 ? RQ_F32 : x_dt, d);
            reorder_pairs(d, pr);
            const int off = e < npc ? slot * MP * kWideRow + (e >> 7) * kWideRow + (e & 127) * 8
                                    : L::DUMMY;
            *(u32x4_t*)&xring[off] = u32x4_t{pr[0], pr[1], pr[2], pr[3]};
        }
    };
    const bool whole = XP || niter <= 2;  // both chunks staged up front
    {
        XRaw xr0[XQ], xr1[XQ];
        load_chunk(0, xr0);
        load_chunk(whole ? 1 : 0, xr1);  // streaming: chunk 0 again (slot 0 is written twice)
        // rows M..MP-1 of both slots and the zero line
        const int zr = (MP - M) * (kWideRow / 8);
        for (int e = threadIdx.x; e < 2 * zr; e += kBlock) {
            const int slot = e >= zr, r = e - slot * zr;
            *(u32x4_t*)&xring[slot * MP * kWideRow + M * kWideRow + r * 8] = u32x4_t{0u, 0u, 0u, 0u};
        }
        if constexpr (MP == 8) {
            for (int e = threadIdx.x; e < kWideKC / 8; e += kBlock)
                *(u32x4_t*)&xring[L::ZERO + e * 8] = u32x4_t{0u, 0u, 0u, 0u};
        }
        store_chunk(0, xr0);
        store_chunk(whole ? 1 : 0, xr1);
    }
    __syncthreads();

    // ---- per-lane constants
    const PairConsts kc = pair_consts();
    constexpr uint32_t kOne = 0x3F803F80u;  // bf16 1.0 pairs
    const bf16x8_t ones = as_bf16x8(kOne, kOne, kOne, kOne);
    // A fragment addresses (elements) in slot 0 and slot 1
    uint32_t a_base[2];
    if constexpr (MP == 8) {
        // lane (lg, lr): A row lr of slot lr/8 has x[lr % 8] on the pieces of
        // lane groups with (lg & 1) == lr/8: piece 8 (lg >> 1) of unit lg & 1
        const bool act = ((lr >> 3) == (lg & 1)) && (lr & 7) < M;
        const uint32_t col = (uint32_t)(64 * (lg & 1) + 8 * (lg >> 1));
#pragma unroll
        for (int s = 0; s < 2; ++s)
            a_base[s] = act ? (uint32_t)(s * MP * kWideRow + (lr & 7) * kWideRow) + col
                            : (uint32_t)L::ZERO + col;
    } else {
#pragma unroll
        for (int s = 0; s < 2; ++s) a_base[s] = (uint32_t)(s * MP * kWideRow + lr * kWideRow + lg * 8);
    }
    uint8_t* win = wins + wave * W::WAVE_BYTES;
    uint8_t* win_w = win + lr * W::ROWB + (lg & 1) * W::WW + (lg >> 1) * (W::WW / 2);
    const uint8_t* win_r = win + lr * W::ROWB;

    auto sb_at = [&](int gw, float& s, float& cb) {  // group gw of the window, row lr
        s = raw_to_f32<SDT>(*(const uint16_t*)(win_r + gw * 2));
        const float b = raw_to_f32<SDT>(*(const uint16_t*)(win_r + W::WW + gw * 2));
        cb = (BITS == 8) ? b : fmaf(s, -128.f, b);
    };

    f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
    auto run = [&](auto streaming) {
        for (int it = 0; it < niter; ++it) {
            if constexpr (XP) {
                // rows longer than two chunks: the next pair is staged behind two
                // barriers once every wave is done with the previous one
                if (it > 0 && (it & 1) == 0) {
                    XRaw xa[XQ], xb[XQ];
                    load_chunk(it, xa);
                    load_chunk(it + 1, xb);
                    __syncthreads();
                    store_chunk(0, xa);
                    store_chunk(1, xb);
                    __syncthreads();
                }
            }
            const int itw = it % W::IPW;
            if (itw == 0) {
                // this window of (scale, bias) values into LDS, the next one into registers
                *(win_t*)win_w = wv;  // read below by other lanes of this wave (LDS runs in order)
                __builtin_amdgcn_wave_barrier();
                wv = load_sb_window<GSH, W::WG>(sbrow, part, G, it / W::IPW + 1, P.x);
            }
            XRaw xr[XQ];
            if constexpr (decltype(streaming)::value) load_chunk(it + 1, xr);
            const uint16_t* xs = xring + a_base[it & 1];
#pragma unroll
            for (int t = 0; t < NS; ++t) {
                const int st = it * NS + t;
                load_codes(st + NS - 1, cw[(t + NS - 1) % NS]);
                if (st < nst) {
                    const int gw0 = itw * W::GPI + t * W::GPS;  // first group of the stage in the window
                    uint32_t* w = cw[t];
                    if constexpr (MP == 8) {
                        // (scale, bias) of this lane's groups, read before the MFMAs so
                        // that the LDS latency is hidden: unit 2 Pp + (lg >> 1) of pair Pp
                        constexpr int NG = GSH == 5 ? 4 : 2;
                        float sc[NG], cb[NG];
#pragma unroll
                        for (int q = 0; q < NG; ++q) {
                            const int Pp = GSH == 5 ? q >> 1 : q, unit = 2 * Pp + (lg >> 1);
                            const int g = GSH == 5 ? 2 * unit + (q & 1) : (GSH == 6 ? unit : unit >> 1);
                            sb_at(gw0 + g, sc[q], cb[q]);
                        }
#pragma unroll
                        for (int v = 0; v < 4; ++v)
#pragma unroll
                            for (int p = 0; p < PW; ++p) swap_lane_halves(w[2 * v * PW + p], w[(2 * v + 1) * PW + p]);
                        f32x4_t d[2], xsum[2];
#pragma unroll
                        for (int v = 0; v < 4; ++v) {
                            uint32_t pr[2][4];
                            if constexpr (BITS == 4) {
                                codes4_to_bf16_pairs_x2(w[2 * v], w[2 * v + 1], pr[0], pr[1], kc);
                            } else {
                                codes_to_bf16_pairs<BITS>(w, 2 * v, pr[0], kc);
                                codes_to_bf16_pairs<BITS>(w, 2 * v + 1, pr[1], kc);
                            }
#pragma unroll
                            for (int Pp = 0; Pp < 2; ++Pp) {
                                const u32x4_t av = *(const u32x4_t*)&xs[t * 256 + 128 * Pp + 16 * v];
                                const bf16x8_t a = as_bf16x8(av[0], av[1], av[2], av[3]);
                                const f32x4_t z = f32x4_t{0.f, 0.f, 0.f, 0.f};
                                const bool first = GSH == 5 ? (v & 1) == 0 : v == 0;
                                d[Pp] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                    a, as_bf16x8(pr[Pp][0], pr[Pp][1], pr[Pp][2], pr[Pp][3]),
                                    first ? z : d[Pp], 0, 0, 0);
                                xsum[Pp] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, first ? z : xsum[Pp], 0, 0, 0);
                            }
                            // gs 32: pieces 2v + b of v < 2 are a unit's first run
                            if (GSH != 5 ? v == 3 : (v & 1) == 1) {
#pragma unroll
                                for (int Pp = 0; Pp < 2; ++Pp) {
                                    const int q = GSH == 5 ? 2 * Pp + (v >> 1) : Pp;
#pragma unroll
                                    for (int i = 0; i < 4; ++i)
                                        acc[i] = fmaf(sc[q], d[Pp][i], fmaf(cb[q], xsum[Pp][i], acc[i]));
                                }
                            }
                        }
                    } else {
#pragma unroll
                        for (int h = 0; h < 2; ++h)
#pragma unroll
                            for (int p = 0; p < PW; ++p)
                                transpose_lane_groups(w[h * BITS + p], w[h * BITS + PW + p],
                                                      w[h * BITS + 2 * PW + p], w[h * BITS + 3 * PW + p]);
                        float sc[W::GPS], cb[W::GPS];
#pragma unroll
                        for (int q = 0; q < W::GPS; ++q) sb_at(gw0 + q, sc[q], cb[q]);
                        f32x4_t d = f32x4_t{0.f, 0.f, 0.f, 0.f}, xsum = d;
#pragma unroll
                        for (int u = 0; u < 8; ++u) {  // run u = 2 t2 + h of the stage
                            const int t2 = u >> 1, h = u & 1;
                            uint32_t pr[4];
                            codes_to_bf16_pairs<BITS>(w + h * BITS, t2, pr, kc);
                            const u32x4_t av = *(const u32x4_t*)&xs[t * 256 + 32 * u];
                            const bf16x8_t a = as_bf16x8(av[0], av[1], av[2], av[3]);
                            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                a, as_bf16x8(pr[0], pr[1], pr[2], pr[3]), d, 0, 0, 0);
                            xsum = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, xsum, 0, 0, 0);
                            const int gi = (32 * u) >> GSH;
                            if (u == 7 || ((32 * (u + 1)) >> GSH) != gi) {  // the group ends with this run
#pragma unroll
                                for (int i = 0; i < 4; ++i)
                                    acc[i] = fmaf(sc[gi], d[i], fmaf(cb[gi], xsum[i], acc[i]));
                                d = f32x4_t{0.f, 0.f, 0.f, 0.f};
                                xsum = d;
                            }
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (decltype(streaming)::value) {
                store_chunk((it + 1) & 1, xr);  // that slot was last read before the previous barrier
                __syncthreads();
            }
        }
    };
    if constexpr (XP) {
        run(std::integral_constant<bool, false>());
    } else {
        if (whole) run(std::integral_constant<bool, false>());
        else run(std::integral_constant<bool, true>());
    }

    const int64_t row = row0 + lr;
    if constexpr (MP == 8) {
        // rows m = 4 (lg & 1) + i: lane groups g and g ^ 2 hold the two slots' parts
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = acc[i] + __shfl_xor(acc[i], 32, 64);
            const int m = 4 * lg + i;
            if (lg < 2 && m < M && row < R) store_dt(P.y, y_dt, (int64_t)m * R + row, v);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * lg + i;
            if (m < M && row < R) store_dt(P.y, y_dt, (int64_t)m * R + row, acc[i]);
        }
    }
}

template <int BITS, int SDT, int MP, int GSH, bool XF32>
__global__ __launch_bounds__(kBlock) void qmv_wide_inline(const QmvArgs args) {
    const int bid = blockIdx.x;
    int lo = 0, hi = args.n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (args.block_start[mid] <= bid) lo = mid; else hi = mid - 1;
    }
    qmv_wide_body<BITS, SDT, MP, GSH, XF32>(args.p[lo], bid - args.block_start[lo], args.m,
                                            args.x_dt, args.y_dt);
}

template <int BITS, int SDT, int MP, int GSH, bool XF32>
__global__ __launch_bounds__(kBlock) void qmv_wide_table(const rq::QmvTable a) {
    const uint32_t e = a.blocks[blockIdx.x];
    const rq_problem P = a.descs[e >> 16];
    qmv_wide_body<BITS, SDT, MP, GSH, XF32>(P, (int)(e & 0xffffu), a.m, a.x_dt, a.y_dt);
}

// F is called with integral_constant-typed (SDT, MP, GSH, XF32).
template <typename F>
hipError_t wide_dispatch(int sb_dt, int64_t m, int gs, int x_dt, F&& f) {
    const int gsh = __builtin_ctz(gs);
    typedef std::integral_constant<int, RQ_BF16> BF;
    typedef std::integral_constant<int, RQ_F16> FH;
    typedef std::integral_constant<bool, true> XF;
    typedef std::integral_constant<bool, false> XH;
#define RQ_W_GSH(SD, MPV, XV)                                                          \
    switch (gsh) {                                                                     \
        case 5: return f(SD(), std::integral_constant<int, MPV>(),                     \
                         std::integral_constant<int, 5>(), XV());                      \
        case 6: return f(SD(), std::integral_constant<int, MPV>(),                     \
                         std::integral_constant<int, 6>(), XV());                      \
        case 7: return f(SD(), std::integral_constant<int, MPV>(),                     \
                         std::integral_constant<int, 7>(), XV());                      \
        default: return hipErrorInvalidValue;                                          \
    }
#define RQ_W_X(SD, MPV)                                  \
    if (x_dt == RQ_F32) { RQ_W_GSH(SD, MPV, XF) }        \
    RQ_W_GSH(SD, MPV, XH)
#define RQ_W_MP(SD)                      \
    if (m <= 8) { RQ_W_X(SD, 8) }        \
    RQ_W_X(SD, 16)
    if (sb_dt == RQ_BF16) { RQ_W_MP(BF) }
    RQ_W_MP(FH)
#undef RQ_W_MP
#undef RQ_W_X
#undef RQ_W_GSH
}

// Template dispatch shared by both launch forms: F is called with
// integral_constant-typed (SDT, NMC, MI, GSH).
template <typename F>
hipError_t stream_dispatch(int sb_dt, int64_t m, int gs, F&& f) {
    const int gsh = __builtin_ctz(gs);
    int nmc = (int)((m + 3) / 4);  // four activation rows per pass
    nmc = nmc <= 1 ? 1 : (nmc <= 2 ? 2 : 4);
    const int mi = nmc > 1 ? 4 : (m >= 3 ? 4 : (int)m);
    typedef std::integral_constant<int, RQ_BF16> BF;
    typedef std::integral_constant<int, RQ_F16> FH;
#define RQ_S_GSH(SD, N, I)                                                                        \
    switch (gsh) {                                                                                \
        case 5: return f(SD(), std::integral_constant<int, N>(), std::integral_constant<int, I>(), \
                         std::integral_constant<int, 5>());                                       \
        case 6: return f(SD(), std::integral_constant<int, N>(), std::integral_constant<int, I>(), \
                         std::integral_constant<int, 6>());                                       \
        case 7: return f(SD(), std::integral_constant<int, N>(), std::integral_constant<int, I>(), \
                         std::integral_constant<int, 7>());                                       \
        default: return hipErrorInvalidValue;                                                     \
    }
#define RQ_S_NMI(SD)                                 \
    switch (nmc * 8 + mi) {                          \
        case 9: RQ_S_GSH(SD, 1, 1)                   \
        case 10: RQ_S_GSH(SD, 1, 2)                  \
        case 12: RQ_S_GSH(SD, 1, 4)                  \
        default: return hipErrorInvalidValue;        \
    }
    if (sb_dt == RQ_BF16) { RQ_S_NMI(BF) }
    RQ_S_NMI(FH)
#undef RQ_S_NMI
#undef RQ_S_GSH
}

hipError_t launch_stream_inline(const QmvArgs& a, int blocks, int sb_dt, int gs, size_t lds,
                                hipStream_t stream) {
    if (a.m > kStreamSlotsMax) {
        if constexpr (RQ_BITS == 4 || RQ_BITS == 8) {
            return wide_dispatch(sb_dt, a.m, gs, a.x_dt, [&](auto sd, auto mp, auto gsh, auto xf) {
                hipLaunchKernelGGL((qmv_wide_inline<RQ_BITS, decltype(sd)::value, decltype(mp)::value,
                                                    decltype(gsh)::value, decltype(xf)::value>),
                                   dim3(blocks), dim3(kBlock), 0, stream, a);
                return hipGetLastError();
            });
        }
        return hipErrorInvalidValue;
    }
    return stream_dispatch(sb_dt, a.m, gs, [&](auto sd, auto nmc, auto mi, auto gsh) {
        hipLaunchKernelGGL((qmv_stream_inline<RQ_BITS, decltype(sd)::value, decltype(nmc)::value,
                                              decltype(mi)::value, decltype(gsh)::value>),
                           dim3(blocks), dim3(kBlock), lds, stream, a);
        return hipGetLastError();
    });
}

// The split GEMV's instantiations: m <= 4 activation rows in one pass (MI
// 1, 2, 4: slices of up to 4, 4 and 2 stages) and 4 < m <= 8 in two (MI 4,
// up to 2 stages); 8-bit codes (twice the registers per stage) one step
// less where more would spill.  "Pass code" pc = 8 * NMC + MI.
constexpr int split_max_nsw(int pc) {
    return RQ_BITS == 8 ? (pc == 9 ? 4 : (pc == 20 ? 1 : 2)) : (pc == 9 || pc == 10 ? 4 : 2);
}
inline int split_pass_code(int64_t m) { return m > 4 ? 20 : (m >= 3 ? 12 : 8 + (int)m); }

// Folding a small launch (m <= 2): W [R, K] read as [2R, K/2] -- the same bytes, row
// r's halves are rows 2r and 2r + 1, and so are its (scale, bias) values --
// against x read as [2m, K/2] (x row m's halves are rows 2m, 2m + 1).  Output
// (2m + p, 2r + q) is half p of x row m against half q of weight row r; the
// kernel stores half 0 + half 1 of the p == q ones (QmvArgs::fold).  Twice
// the 16-row tiles, each over half the stages: for launches that leave most
// CUs idle ([2048, 8192]: 128 tiles of 32 stages become 256 of 16).
#ifndef RQ_QMV_FOLD
#define RQ_QMV_FOLD 1
#endif
constexpr int64_t kFoldMaxBlocks = 128;  // tiles of a launch that folds, at most

inline rq_problem split_fold(rq_problem p) {
    p.rows *= 2;
    p.cols /= 2;
    return p;
}

// LDS a split-GEMV block may take when the launch has at most one block per
// CU (then nothing shares the CU's 160 KB): [2048, 8192] at m = 8 stages 8
// rows x 512 columns of x per wave, 16 waves, ~145 KB.
constexpr int kSplitLdsOneBlock = 152 * 1024;
constexpr int64_t kSplitOneBlockMax = 256;  // blocks of a launch that fit one per CU

bool split_covers(const rq_problem& p, int sb_dt, int64_t m, int gs, int budget) {
    if (sb_dt == RQ_F32 || m < 1 || m > 8 || p.cols % 256 != 0 || p.rows < 1) return false;
    const int nsw = split_nsw(p.cols);
    if (nsw == 0 || nsw > split_max_nsw(split_pass_code(m))) return false;
    const int gsh = __builtin_ctz(gs);
    const int sb1 = (256 >> gsh) * 2;  // bytes of one array per row and stage
    const int sbh = nsw * sb1 / 2;     // (scale, bias) bytes one lane loads
    const int sbw = sbh < sb1 ? sbh : (sb1 < 16 ? sb1 : 16);
    const int64_t row_bytes = (p.cols >> gsh) * 2;
    const int ks = (int)(((p.cols >> 8) + nsw - 1) / nsw);
    const uintptr_t code_align = (RQ_BITS & 1) ? 7 : 15;
    return row_bytes % sbw == 0 && (((uintptr_t)p.scales | (uintptr_t)p.biases) % sbw) == 0 &&
           ((uintptr_t)p.w_q & code_align) == 0 && ((uintptr_t)p.x & 15) == 0 &&
           (int64_t)ks * split_wave_bytes((int)m, nsw, gsh, RQ_BITS) <= budget;
}

hipError_t launch_split(const QmvArgs& a, int blocks, int64_t cols, int sb_dt, int gs,
                        hipStream_t stream) {
    const int nsw = split_nsw(cols);
    const int ks = (int)(((cols >> 8) + nsw - 1) / nsw);
    const int gsh = __builtin_ctz(gs);
    // the kernel lays out its wave regions for exactly a.m activation rows
    const size_t lds = (size_t)ks * split_wave_bytes(a.m, nsw, gsh, RQ_BITS);
    auto go = [&](auto sd, auto nmcc, auto mic, auto gshc, auto nswc) {
        constexpr int NMC = decltype(nmcc)::value, MI = decltype(mic)::value;
        constexpr int NSW = decltype(nswc)::value;
        if constexpr (NSW <= split_max_nsw(8 * NMC + MI)) {
            hipLaunchKernelGGL((qmv_split<RQ_BITS, decltype(sd)::value, NMC, MI, decltype(gshc)::value,
                                          NSW>),
                               dim3(blocks), dim3(64 * ks), lds, stream, a);
            return hipGetLastError();
        }
        return hipErrorInvalidValue;
    };
    typedef std::integral_constant<int, RQ_BF16> BF;
    typedef std::integral_constant<int, RQ_F16> FH;
    auto by_nsw = [&](auto sd, auto nmcc, auto mic, auto gshc) {
        switch (nsw) {
            case 1: return go(sd, nmcc, mic, gshc, std::integral_constant<int, 1>());
            case 2: return go(sd, nmcc, mic, gshc, std::integral_constant<int, 2>());
            case 4: return go(sd, nmcc, mic, gshc, std::integral_constant<int, 4>());
            default: return hipErrorInvalidValue;
        }
    };
    auto by_gs = [&](auto sd, auto nmcc, auto mic) {
        switch (gsh) {
            case 5: return by_nsw(sd, nmcc, mic, std::integral_constant<int, 5>());
            case 6: return by_nsw(sd, nmcc, mic, std::integral_constant<int, 6>());
            case 7: return by_nsw(sd, nmcc, mic, std::integral_constant<int, 7>());
            default: return hipErrorInvalidValue;
        }
    };
    typedef std::integral_constant<int, 1> C1;
    typedef std::integral_constant<int, 2> C2;
    auto by_m = [&](auto sd) {
        switch (split_pass_code(a.m)) {
            case 9: return by_gs(sd, C1(), std::integral_constant<int, 1>());
            case 10: return by_gs(sd, C1(), std::integral_constant<int, 2>());
            case 12: return by_gs(sd, C1(), std::integral_constant<int, 4>());
            case 20: return by_gs(sd, C2(), std::integral_constant<int, 4>());
            default: return hipErrorInvalidValue;
        }
    };
    return sb_dt == RQ_BF16 ? by_m(BF()) : by_m(FH());
}

hipError_t launch_stream_table(const rq::QmvTable& a, int blocks, int sb_dt, int gs, size_t lds,
                               hipStream_t stream) {
    if (a.m > kStreamSlotsMax) {
        if constexpr (RQ_BITS == 4 || RQ_BITS == 8) {
            return wide_dispatch(sb_dt, a.m, gs, a.x_dt, [&](auto sd, auto mp, auto gsh, auto xf) {
                hipLaunchKernelGGL((qmv_wide_table<RQ_BITS, decltype(sd)::value, decltype(mp)::value,
                                                   decltype(gsh)::value, decltype(xf)::value>),
                                   dim3(blocks), dim3(kBlock), 0, stream, a);
                return hipGetLastError();
            });
        }
        return hipErrorInvalidValue;
    }
    return stream_dispatch(sb_dt, a.m, gs, [&](auto sd, auto nmc, auto mi, auto gsh) {
        hipLaunchKernelGGL((qmv_stream_table<RQ_BITS, decltype(sd)::value, decltype(nmc)::value,
                                             decltype(mi)::value, decltype(gsh)::value>),
                           dim3(blocks), dim3(kBlock), lds, stream, a);
        return hipGetLastError();
    });
}
}  // namespace

namespace rq {

#define RQ_CAT2(a, b) a##b
#define RQ_CAT(a, b) RQ_CAT2(a, b)

// One launch over problems[0..n) that all share cols (so LDS staging is sized
// exactly for them).
static hipError_t launch_bucket(const rq_problem* const* probs, int n, int x_dt, int sb_dt,
                                int y_dt, int64_t m, int gs, hipStream_t stream) {
    // from here on m counts MFMA activation rows: with the hi/lo split of
    // fp32 / f16 x, twice the problem's rows
    const int xsplit = qmv_xsplit(x_dt, m) ? 1 : 0;
    m = qmv_rows(x_dt, m);
    const int gs_shift = __builtin_ctz(gs);
    const int MC = 16 >> (7 - gs_shift);
    int nmc = (int)((m + MC - 1) / MC);
    nmc = nmc <= 1 ? 1 : (nmc <= 2 ? 2 : 4);
    const int64_t K = probs[0]->cols;

    // The total number of 16-row blocks picks the organisation: big launches
    // give every wave RQ_QMV_BIG_RB row blocks of its own, medium ones one,
    // and small ones let the four waves of a block split K so that more waves
    // stream at once.
    int64_t rowblocks = 0;
    for (int i = 0; i < n; ++i) rowblocks += (probs[i]->rows + 15) / 16;
    const int cfg = rowblocks >= RQ_QMV_BIG_MIN ? 2 : (rowblocks >= 2048 ? 1 : 0);
    // Small launches: the split GEMV (one memory round trip per launch).
    bool split = cfg == 0 && RQ_QMV_SPLIT;
    // Launches of at most kFoldMaxBlocks tiles fold (split_fold): twice the
    // tiles, each over half of K.  Measured per launch: faster at m = 1 (e.g.
    // [2048, 8192] 7.04 -> 5.77 us, [2048, 2048] 4.44 -> 4.19) and at m = 2
    // with K >= 4096; at m = 2, K = 2048 and at m >= 3 (two passes of 8
    // activation rows at m = 4) slower.
    bool fold = split && RQ_QMV_FOLD && !xsplit && (m == 1 || (m == 2 && K >= 4096)) &&
                K % 512 == 0 && rowblocks <= kFoldMaxBlocks;
    for (int i = 0; i < n && fold; ++i)
        fold = split_covers(split_fold(*probs[i]), sb_dt, 2 * m, gs,
                            2 * rowblocks <= kSplitOneBlockMax ? kSplitLdsOneBlock : kLdsBudget);
    const int split_budget = rowblocks <= kSplitOneBlockMax ? kSplitLdsOneBlock : kLdsBudget;
    for (int i = 0; i < n && split && !fold; ++i)
        split = split_covers(*probs[i], sb_dt, m, gs, split_budget);
    if (split) {
        for (int base = 0; base < n; base += RQ_MAX_GROUPED) {
            const int cnt = (n - base) < RQ_MAX_GROUPED ? (n - base) : RQ_MAX_GROUPED;
            QmvArgs a;
            std::memset(&a, 0, sizeof(a));
            int64_t blocks = 0;
            for (int i = 0; i < cnt; ++i) {
                a.p[i] = fold ? split_fold(*probs[base + i]) : *probs[base + i];
                a.block_start[i] = (int)blocks;
                blocks += (a.p[i].rows + 15) / 16;
            }
            a.block_start[cnt] = (int)blocks;
            a.n = cnt;
            a.m = (int)(fold ? 2 * m : m);
            a.gs_shift = gs_shift;
            a.x_dt = x_dt;
            a.y_dt = y_dt;
            a.xsplit = xsplit;
            a.fold = fold ? 1 : 0;
            hipError_t e = launch_split(a, (int)blocks, fold ? K / 2 : K, sb_dt, gs, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    bool streamed = cfg >= 1 && RQ_QMV_STREAM;
    for (int i = 0; i < n && streamed; ++i) streamed = qmv_stream_covers(*probs[i], sb_dt, m, gs, RQ_BITS);
    if (streamed) {
        const size_t lds = qmv_stream_lds(m, K, gs, RQ_BITS);
        for (int base = 0; base < n; base += RQ_MAX_GROUPED) {
            const int cnt = (n - base) < RQ_MAX_GROUPED ? (n - base) : RQ_MAX_GROUPED;
            QmvArgs a;
            std::memset(&a, 0, sizeof(a));
            int64_t blocks = 0;
            for (int i = 0; i < cnt; ++i) {
                a.p[i] = *probs[base + i];
                a.block_start[i] = (int)blocks;
                blocks += (probs[base + i]->rows + kQmvRowsPerBlock - 1) / kQmvRowsPerBlock;
            }
            a.block_start[cnt] = (int)blocks;
            a.n = cnt;
            a.m = (int)m;
            a.gs_shift = gs_shift;
            a.x_dt = x_dt;
            a.y_dt = y_dt;
            a.xsplit = xsplit;
            if (blocks == 0) continue;
            hipError_t e = launch_stream_inline(a, (int)blocks, sb_dt, gs, lds, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const int RB = cfg == 2 ? RQ_QMV_BIG_RB : 1;
    const int rows_per_block = cfg == 0 ? 16 * RB : 16 * RB * kWaves;
    // LDS staging: a zero line, activations [m][K] as bf16, their group sums
    // [m][K/gs] fp32, then the block's (scale, bias) pairs.
    const size_t sbsz = sb_dt == RQ_F32 ? 8 : 4;
    const size_t lds = 64 + (((size_t)m * K * 2 + 15) & ~(size_t)15) +
                       (((size_t)m * (K / gs) * 4 + 15) & ~(size_t)15) +
                       (size_t)rows_per_block * (K / gs) * sbsz;
    const bool xlds = lds <= (size_t)kLdsBudget;
    const size_t dyn = xlds ? lds : 0;

    for (int base = 0; base < n; base += RQ_MAX_GROUPED) {
        const int cnt = (n - base) < RQ_MAX_GROUPED ? (n - base) : RQ_MAX_GROUPED;
        QmvArgs a;
        std::memset(&a, 0, sizeof(a));
        int64_t blocks = 0;
        for (int i = 0; i < cnt; ++i) {
            a.p[i] = *probs[base + i];
            a.block_start[i] = (int)blocks;
            blocks += (probs[base + i]->rows + rows_per_block - 1) / rows_per_block;
        }
        a.block_start[cnt] = (int)blocks;
        a.n = cnt;
        a.m = (int)m;
        a.gs_shift = gs_shift;
        a.x_dt = x_dt;
        a.y_dt = y_dt;
        a.xsplit = xsplit;
        a.sb_vec = 1;
        for (int i = 0; i < cnt; ++i)
            a.sb_vec &= (((uintptr_t)a.p[i].scales | (uintptr_t)a.p[i].biases) & 15) == 0;
        if (blocks == 0) continue;
        hipError_t e;
        if (cfg == 2) e = launch_cfg<RQ_QMV_BIG_RB, 1>(a, sb_dt, nmc, xlds, (int)blocks, dyn, stream);
        else if (cfg == 1) e = launch_cfg<1, 1>(a, sb_dt, nmc, xlds, (int)blocks, dyn, stream);
        else e = launch_cfg<1, kWaves>(a, sb_dt, nmc, xlds, (int)blocks, dyn, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

#if RQ_BITS == 4  // bit-width independent helpers: defined in one unit only
size_t qmv_stream_lds(int64_t m, int64_t cols, int gs, int bits) {
    if (m > kStreamSlotsMax) return 0;  // the wide kernel's LDS is static
    const int wave_bytes = gs == 32 ? StreamWin<5>::WAVE_BYTES
                         : (gs == 64 ? StreamWin<6>::WAVE_BYTES : StreamWin<7>::WAVE_BYTES);
    const int xg = gs < 64 ? gs : 64;  // elements per activation sum
    const size_t nsum = bits == 3 ? 2 : 1;  // 3-bit: sums over all and over low-half positions
    return 2 * kZeroElems + (((size_t)m * cols * 2 + 15) & ~(size_t)15) +
           nsum * (((size_t)m * (cols / xg) * 4 + 15) & ~(size_t)15) + 4 * (size_t)wave_bytes;
}
bool qmv_stream_covers(const rq_problem& p, int sb_dt, int64_t m, int gs, int bits) {
    const bool layout = sb_dt != RQ_F32 && p.cols % 512 == 0 &&
                        p.rows <= (int64_t)65536 * kQmvRowsPerBlock &&
                        (((uintptr_t)p.scales | (uintptr_t)p.biases) & 15) == 0;
    if (m > kStreamSlotsMax)  // the wide kernel (static LDS, chunked x)
        return RQ_QMV_WIDE && layout && m <= 16 && (bits == 4 || bits == 8);
    return layout && qmv_stream_lds(m, p.cols, gs, bits) <= (size_t)kQmvLdsBudget;
}
#endif

hipError_t RQ_CAT(launch_qmv_table_b, RQ_BITS)(const QmvTable& t, int blocks, int sb_dt, int gs,
                                               size_t lds, hipStream_t stream) {
    return launch_stream_table(t, blocks, sb_dt, gs, lds, stream);
}

hipError_t RQ_CAT(launch_qmv_b, RQ_BITS)(const rq_problem* problems, int n, int x_dt, int sb_dt,
                                         int y_dt, int64_t m, int gs, hipStream_t stream) {
    // Problems are bucketed by cols (in order of first appearance): each
    // bucket is launched with LDS staging sized for its own K.
    std::vector<const rq_problem*> order;
    std::vector<int64_t> seen;
    order.reserve(n);
    for (int i = 0; i < n; ++i) {
        bool dup = false;
        for (int64_t c : seen) dup |= (c == problems[i].cols);
        if (dup) continue;
        seen.push_back(problems[i].cols);
        const size_t start = order.size();
        for (int k = i; k < n; ++k)
            if (problems[k].cols == problems[i].cols && problems[k].rows > 0)
                order.push_back(&problems[k]);
        if (order.size() > start) {
            hipError_t e = launch_bucket(order.data() + start, (int)(order.size() - start), x_dt,
                                         sb_dt, y_dt, m, gs, stream);
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

}  // namespace rq
