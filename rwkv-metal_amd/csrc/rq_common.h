// rq_common.h -- device helpers shared by the gfx950 kernels of librwkvq_hip.
//
// Storage types: bf16 and f16 live in 16-bit words, f32 in float.  All
// arithmetic is fp32.  Conversions to bf16 are round-to-nearest-even, the
// same rounding MLX applies when it casts fp32 results to bfloat16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/rwkvq.h"

#define RQ_DEV __device__ __forceinline__

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------ conversions

RQ_DEV float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
RQ_DEV uint32_t f32_to_bf16_bits(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two fp32 values -> one dword holding (bf16(lo), bf16(hi)), RNE.
RQ_DEV uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

RQ_DEV float f16_bits_to_f32(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
    return (float)v;
}
RQ_DEV uint32_t f32_to_f16_bits(float f) {
    _Float16 v = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
    return (uint32_t)__builtin_bit_cast(uint16_t, v);
}

// value of v after a cast to dtype dt (runtime dtype)
RQ_DEV float round_to_dt(int dt, float v) {
    if (dt == RQ_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
    if (dt == RQ_F16) return f16_bits_to_f32(f32_to_f16_bits(v));
    return v;
}

// Load element i of a buffer of runtime dtype dt as fp32.
RQ_DEV float load_dt(const void* p, int dt, int64_t i) {
    if (dt == RQ_F32) return ((const float*)p)[i];
    uint32_t h = ((const uint16_t*)p)[i];
    return dt == RQ_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

RQ_DEV void store_dt(void* p, int dt, int64_t i, float v) {
    if (dt == RQ_F32) {
        ((float*)p)[i] = v;
    } else if (dt == RQ_BF16) {
        ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16_bits(v);
    } else {
        ((uint16_t*)p)[i] = (uint16_t)f32_to_f16_bits(v);
    }
}

// Compile-time dtype traits for the activation/weight operand.
template <int DT>
struct dt_traits;
template <>
struct dt_traits<RQ_BF16> {
    typedef uint16_t storage;
    static RQ_DEV float to_f32(storage h) { return bf16_bits_to_f32(h); }
    static RQ_DEV storage from_f32(float f) { return (storage)f32_to_bf16_bits(f); }
};
template <>
struct dt_traits<RQ_F16> {
    typedef uint16_t storage;
    static RQ_DEV float to_f32(storage h) { return f16_bits_to_f32(h); }
    static RQ_DEV storage from_f32(float f) { return (storage)f32_to_f16_bits(f); }
};
template <>
struct dt_traits<RQ_F32> {
    typedef float storage;
    static RQ_DEV float to_f32(storage h) { return h; }
    static RQ_DEV storage from_f32(float f) { return f; }
};

// Load 32 consecutive elements of dtype DT (16-byte aligned) as fp32.
template <int DT>
RQ_DEV void load32_f32(const void* base, int64_t elem_off, float* out) {
    if constexpr (DT == RQ_F32) {
        const uint4* p = (const uint4*)((const float*)base + elem_off);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint4 v = p[i];
            out[4 * i + 0] = __uint_as_float(v.x);
            out[4 * i + 1] = __uint_as_float(v.y);
            out[4 * i + 2] = __uint_as_float(v.z);
            out[4 * i + 3] = __uint_as_float(v.w);
        }
    } else {
        const uint4* p = (const uint4*)((const uint16_t*)base + elem_off);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint4 v = p[i];
            uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                out[8 * i + 2 * j + 0] = dt_traits<DT>::to_f32((uint16_t)(w[j] & 0xffffu));
                out[8 * i + 2 * j + 1] = dt_traits<DT>::to_f32((uint16_t)(w[j] >> 16));
            }
        }
    }
}

// ------------------------------------------------------------- bitstream

// A "run" is 32 consecutive codes of a row.  32*BITS bits = BITS whole
// words, so runs start on word boundaries and never straddle a group
// (group_size is a multiple of 32).  Code j of a run sits at bit j*BITS of
// the run's little-endian bitstream and may cross into the next word.
template <int BITS>
RQ_DEV uint32_t run_code(const uint32_t* words, int j) {
    const int bit = j * BITS;
    const int w = bit >> 5;
    const int off = bit & 31;
    const uint32_t mask = (1u << BITS) - 1u;
    if (off + BITS <= 32) return (words[w] >> off) & mask;
    // funnel shift across the word boundary
    return (uint32_t)((((uint64_t)words[w + 1] << 32) | words[w]) >> off) & mask;
}

template <int BITS>
RQ_DEV void run_pack(const uint32_t* codes, uint32_t* words) {
#pragma unroll
    for (int w = 0; w < BITS; ++w) words[w] = 0u;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const int bit = j * BITS;
        const int w = bit >> 5;
        const int off = bit & 31;
        words[w] |= codes[j] << off;
        if (off + BITS > 32) words[w + 1] |= codes[j] >> (32 - off);
    }
}

// Load the BITS words of one run (4-byte aligned; 16-byte aligned when
// BITS is 4 or 8).
template <int BITS>
RQ_DEV void load_run(const uint32_t* p, uint32_t* words) {
    if constexpr (BITS == 4) {
        uint4 v = *(const uint4*)p;
        words[0] = v.x; words[1] = v.y; words[2] = v.z; words[3] = v.w;
    } else if constexpr (BITS == 8) {
        uint4 v0 = ((const uint4*)p)[0];
        uint4 v1 = ((const uint4*)p)[1];
        words[0] = v0.x; words[1] = v0.y; words[2] = v0.z; words[3] = v0.w;
        words[4] = v1.x; words[5] = v1.y; words[6] = v1.z; words[7] = v1.w;
    } else if constexpr (BITS == 2) {
        uint2 v = *(const uint2*)p;
        words[0] = v.x; words[1] = v.y;
    } else {
#pragma unroll
        for (int w = 0; w < BITS; ++w) words[w] = p[w];
    }
}

template <int BITS>
RQ_DEV void store_run(uint32_t* p, const uint32_t* words) {
    if constexpr (BITS == 4) {
        *(uint4*)p = make_uint4(words[0], words[1], words[2], words[3]);
    } else if constexpr (BITS == 8) {
        ((uint4*)p)[0] = make_uint4(words[0], words[1], words[2], words[3]);
        ((uint4*)p)[1] = make_uint4(words[4], words[5], words[6], words[7]);
    } else if constexpr (BITS == 2) {
        *(uint2*)p = make_uint2(words[0], words[1]);
    } else {
#pragma unroll
        for (int w = 0; w < BITS; ++w) p[w] = words[w];
    }
}

// Dispatch a runtime bits value to a template functor call.
#define RQ_DISPATCH_BITS(bits, BITS_CONST, ...)                   \
    switch (bits) {                                               \
        case 2: { constexpr int BITS_CONST = 2; __VA_ARGS__; } break; \
        case 3: { constexpr int BITS_CONST = 3; __VA_ARGS__; } break; \
        case 4: { constexpr int BITS_CONST = 4; __VA_ARGS__; } break; \
        case 5: { constexpr int BITS_CONST = 5; __VA_ARGS__; } break; \
        case 6: { constexpr int BITS_CONST = 6; __VA_ARGS__; } break; \
        case 8: { constexpr int BITS_CONST = 8; __VA_ARGS__; } break; \
        default: break;                                           \
    }

#define RQ_DISPATCH_DT(dt, DT_CONST, ...)                                  \
    switch (dt) {                                                          \
        case RQ_BF16: { constexpr int DT_CONST = RQ_BF16; __VA_ARGS__; } break; \
        case RQ_F16: { constexpr int DT_CONST = RQ_F16; __VA_ARGS__; } break;   \
        case RQ_F32: { constexpr int DT_CONST = RQ_F32; __VA_ARGS__; } break;   \
        default: break;                                                    \
    }
