/*
 * rq_oracle.c -- CPU restatement of the group-affine quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library in rwkv-metal_amd/csrc.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product never does.
 *
 * What it restates (reference = RafaelUI/rwkv-metal, which delegates the
 * arithmetic to the upstream `mlx` package, not vendored):
 *   - rqo_quantize   : mx.quantize(w, group_size, bits), affine mode, as called
 *                      from rwkv_metal/lora/finetune.py:88-89 (nn.quantize) and
 *                      rwkv_metal/lora/lora.py:45-46 (QuantizedLinear.from_linear).
 *                      Per group: fp32 min/max, signed scale chosen by the
 *                      larger-magnitude extreme, that extreme stored exactly as
 *                      the bias at code 0, codes = clip(rint((w-b)/s), 0, 2^b-1).
 *   - rqo_pack/unpack: the LSB-first bitstream rule stated at
 *                      rwkv_metal/lora/rwkvq_native.py:18-33 and executed by
 *                      tests/dev_pack_native_mlx.py:38-57 (code p of a row at
 *                      global bit p*bits, fields cross uint32 words).
 *   - rqo_dequantize : w = scales[g]*code + biases[g] (rwkvq_native.py:9-16,
 *                      mx.dequantize used as ground truth at
 *                      tests/dev_pack_native_mlx.py:70), evaluated as MLX's
 *                      composite ops do: multiply, round to the scales dtype,
 *                      add, round again.
 *   - rqo_qmm        : mx.quantized_matmul(x, w_q, s, b, transpose, gs, bits)
 *                      (rwkvq_native.py:119-122, the VJP w.r.t. x for the QLoRA
 *                      backward is the transpose=False form).  Operands are
 *                      promoted to a common dtype T as MLX does; the weights
 *                      are either exactly rqo_dequantize's values in T (the
 *                      form of MLX's tiled qmm, which dequantizes into T) or,
 *                      with exact_w, scale*code + bias evaluated in double
 *                      with no rounding (the form of MLX's qmv, which applies
 *                      scale and bias to per-group sums of x*code and x);
 *                      products are accumulated in double.
 *   - rqo_qmv_bf16   : the same transpose=1 product organised like MLX's CPU
 *                      qmv (per-group sums of x*code and x, scale and bias
 *                      applied once per group), bf16 in and out; the timed CPU
 *                      baseline.
 *   - rqo_count_ties : how many exact half-integer quotients rqo_quantize
 *                      rounds (where rint and round-half-away would differ).
 *   - rqo_sb6_*      : the rwkv-quant sb6 (K3) decode, dense dequantize and
 *                      the scale/min expansion of the native repack
 *                      (rwkv_metal/lora/rwkvq_kernel.py, rwkvq_linear.py,
 *                      rwkvq_native.py; see the section below).
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off so no FMA contraction changes
 * the quantize arithmetic).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { RQ_BF16 = 0, RQ_F16 = 1, RQ_F32 = 2 };

/* ------------------------------------------------------------------ dtypes */

static float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u); /* round to nearest even */
    return (uint16_t)(u >> 16);
}

static float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    int exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    float f;
    if (exp == 0) {
        f = ldexpf((float)man, -24); /* zero or subnormal */
        if (sign) f = -f;
        return f;
    }
    uint32_t u;
    if (exp == 31) u = sign | 0x7f800000u | (man << 13);
    else u = sign | ((uint32_t)(exp - 15 + 127) << 23) | (man << 13);
    memcpy(&f, &u, 4);
    return f;
}

static uint16_t f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u;
    if (a >= 0x477ff000u) return sign | 0x7c00u; /* rounds to >= 65520: inf */
    if (a < 0x38800000u) {                        /* below 2^-14: subnormal */
        /* value = a_float; subnormal unit is 2^-24 */
        float af;
        memcpy(&af, &a, 4);
        float q = af * 16777216.0f; /* exact scaling by 2^24 */
        float r = rintf(q);          /* round half even */
        return sign | (uint16_t)r;
    }
    uint32_t exp = (a >> 23) - 127 + 15;
    uint32_t man = a & 0x7fffffu;
    uint32_t h = (exp << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* may carry into exp: fine */
    return sign | (uint16_t)h;
}

static float load_el(const void* p, int dt, int64_t i) {
    switch (dt) {
        case RQ_BF16: return bf16_to_f32(((const uint16_t*)p)[i]);
        case RQ_F16: return f16_to_f32(((const uint16_t*)p)[i]);
        default: return ((const float*)p)[i];
    }
}

static void store_el(void* p, int dt, int64_t i, float v) {
    switch (dt) {
        case RQ_BF16: ((uint16_t*)p)[i] = f32_to_bf16(v); break;
        case RQ_F16: ((uint16_t*)p)[i] = f32_to_f16(v); break;
        default: ((float*)p)[i] = v; break;
    }
}

/* value of v after a cast to dtype dt */
static float round_to(int dt, float v) {
    switch (dt) {
        case RQ_BF16: return bf16_to_f32(f32_to_bf16(v));
        case RQ_F16: return f16_to_f32(f32_to_f16(v));
        default: return v;
    }
}

/* MLX type promotion restricted to the floating types used here:
 * equal types stay, anything mixed with f32 is f32, bf16 with f16 is f32. */
int rqo_promote(int a, int b) { return a == b ? a : RQ_F32; }

float rqo_round_bf16(float v) { return round_to(RQ_BF16, v); }
float rqo_round_f16(float v) { return round_to(RQ_F16, v); }

static int valid_bits(int bits) {
    return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8;
}
static int valid_gs(int gs) { return gs == 32 || gs == 64 || gs == 128; }
static int valid_dt(int dt) { return dt == RQ_BF16 || dt == RQ_F16 || dt == RQ_F32; }

/* --------------------------------------------------------------- packing */

/* Code j of a row occupies bits [j*bits, (j+1)*bits) of the row's
 * little-endian bitstream (rwkvq_native.py:18-22). */
void rqo_pack(const uint8_t* codes, int64_t rows, int64_t cols, int bits, uint32_t* wq) {
    const int64_t wpr = cols * bits / 32;
    const uint32_t mask = (1u << bits) - 1u;
    for (int64_t r = 0; r < rows; ++r) {
        uint32_t* out = wq + r * wpr;
        memset(out, 0, (size_t)wpr * 4);
        for (int64_t j = 0; j < cols; ++j) {
            uint32_t c = codes[r * cols + j] & mask;
            int64_t bit = j * bits;
            int64_t w = bit >> 5;
            int off = (int)(bit & 31);
            out[w] |= c << off;
            if (off + bits > 32) out[w + 1] |= c >> (32 - off);
        }
    }
}

void rqo_unpack(const uint32_t* wq, int64_t rows, int64_t cols, int bits, uint8_t* codes) {
    const int64_t wpr = cols * bits / 32;
    const uint32_t mask = (1u << bits) - 1u;
    for (int64_t r = 0; r < rows; ++r) {
        const uint32_t* in = wq + r * wpr;
        for (int64_t j = 0; j < cols; ++j) {
            int64_t bit = j * bits;
            int64_t w = bit >> 5;
            int off = (int)(bit & 31);
            uint64_t win = in[w];
            if (off + bits > 32) win |= (uint64_t)in[w + 1] << 32;
            codes[r * cols + j] = (uint8_t)((win >> off) & mask);
        }
    }
}

/* -------------------------------------------------------------- quantize */

/* One group of gs values (fp32 copies of the inputs) -> codes, scale, bias.
 * The arithmetic and its order follow the affine quantizer of MLX's CPU
 * backend (all single precision, IEEE division, rint = round-half-even). */
/* A quotient that lies exactly half-way between two integers: the one case
 * where rint (half-to-even) and round (half-away-from-zero) differ. */
static int is_half_tie(float v) { return v - floorf(v) == 0.5f; }

/* ties (optional): incremented once per exact half-integer quotient seen by
 * the rounding of q0 or of a code, before clipping. */
static void quantize_group(const float* w, int gs, int bits, uint8_t* codes,
                           float* scale_out, float* bias_out, int64_t* ties) {
    const float n_bins = (float)((1 << bits) - 1);
    const float eps = 1e-7f;
    float w_min = INFINITY, w_max = -INFINITY;
    for (int j = 0; j < gs; ++j) {
        w_max = fmaxf(w_max, w[j]);
        w_min = fminf(w_min, w[j]);
    }
    int side = fabsf(w_min) > fabsf(w_max);
    float scale = fmaxf((w_max - w_min) / n_bins, eps);
    scale = side ? scale : -scale;
    float edge = side ? w_min : w_max;
    const float e = edge / scale;
    if (ties && is_half_tie(e)) ++*ties;
    float q0 = rintf(e);
    float bias = 0.0f;
    if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
    }
    for (int j = 0; j < gs; ++j) {
        const float v = (w[j] - bias) / scale;
        if (ties && is_half_tie(v)) ++*ties;
        float q = rintf(v);
        q = fminf(fmaxf(q, 0.0f), n_bins);
        codes[j] = (uint8_t)q;
    }
    *scale_out = scale;
    *bias_out = bias;
}

int rqo_quantize(const void* w, int w_dt, int64_t rows, int64_t cols, int gs, int bits,
                 uint32_t* wq, void* scales, void* biases) {
    if (!valid_bits(bits) || !valid_gs(gs) || !valid_dt(w_dt)) return -1;
    if (rows < 0 || cols <= 0 || cols % gs != 0) return -1;
    const int64_t G = cols / gs;
    const int64_t wpr = cols * bits / 32;
#pragma omp parallel
    {
        float* buf = (float*)malloc(sizeof(float) * (size_t)gs);
        uint8_t* rowcodes = (uint8_t*)malloc((size_t)cols);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            for (int64_t g = 0; g < G; ++g) {
                for (int j = 0; j < gs; ++j) buf[j] = load_el(w, w_dt, r * cols + g * gs + j);
                float s, b;
                quantize_group(buf, gs, bits, rowcodes + g * gs, &s, &b, NULL);
                store_el(scales, w_dt, r * G + g, s);
                store_el(biases, w_dt, r * G + g, b);
            }
            rqo_pack(rowcodes, 1, cols, bits, wq + r * wpr);
        }
        free(buf);
        free(rowcodes);
    }
    return 0;
}

/* Number of exact half-integer quotients rqo_quantize rounds on w (the q0
 * of each group and every code before clipping).  These are the only values
 * where MLX's CPU rint (half-to-even) and a half-away-from-zero round would
 * give different codes, so a count of zero on a workload means its codes do
 * not depend on that choice. */
int64_t rqo_count_ties(const void* w, int w_dt, int64_t rows, int64_t cols, int gs, int bits) {
    if (!valid_bits(bits) || !valid_gs(gs) || !valid_dt(w_dt)) return -1;
    if (rows < 0 || cols <= 0 || cols % gs != 0) return -1;
    const int64_t G = cols / gs;
    int64_t total = 0;
#pragma omp parallel reduction(+ : total)
    {
        float* buf = (float*)malloc(sizeof(float) * (size_t)gs);
        uint8_t* codes = (uint8_t*)malloc((size_t)gs);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r)
            for (int64_t g = 0; g < G; ++g) {
                for (int j = 0; j < gs; ++j) buf[j] = load_el(w, w_dt, r * cols + g * gs + j);
                float s, b;
                quantize_group(buf, gs, bits, codes, &s, &b, &total);
            }
        free(buf);
        free(codes);
    }
    return total;
}

/* ------------------------------------------------------------ dequantize */

/* ŵ = T(T(code * s) + b) with s, b already in T (two roundings, as MLX's
 * multiply-then-add composition produces). */
static inline float dq_value(uint32_t code, float s, float b, int T) {
    float p = round_to(T, (float)code * s);
    return round_to(T, p + b);
}

/* Dequantize rows [r0, r1) into fp32 values that are exactly representable in
 * T = promote(sb_dt, T_req). */
static void dequant_rows_f32(const uint32_t* wq, const void* scales, const void* biases,
                             int sb_dt, int T, int64_t r, int64_t cols, int gs, int bits,
                             float* out) {
    const int64_t wpr = cols * bits / 32;
    const int64_t G = cols / gs;
    const uint32_t mask = (1u << bits) - 1u;
    const uint32_t* in = wq + r * wpr;
    for (int64_t g = 0; g < G; ++g) {
        float s = round_to(T, load_el(scales, sb_dt, r * G + g));
        float b = round_to(T, load_el(biases, sb_dt, r * G + g));
        for (int j = 0; j < gs; ++j) {
            int64_t k = g * gs + j;
            int64_t bit = k * bits;
            int64_t w = bit >> 5;
            int off = (int)(bit & 31);
            uint64_t win = in[w];
            if (off + bits > 32) win |= (uint64_t)in[w + 1] << 32;
            uint32_t c = (uint32_t)((win >> off) & mask);
            out[k] = dq_value(c, s, b, T);
        }
    }
}

int rqo_dequantize(const uint32_t* wq, const void* scales, const void* biases, int sb_dt,
                   int64_t rows, int64_t cols, int gs, int bits, void* out, int out_dt) {
    if (!valid_bits(bits) || !valid_gs(gs) || !valid_dt(sb_dt) || !valid_dt(out_dt)) return -1;
    if (rows < 0 || cols <= 0 || cols % gs != 0) return -1;
#pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)cols);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            dequant_rows_f32(wq, scales, biases, sb_dt, sb_dt, r, cols, gs, bits, row);
            for (int64_t k = 0; k < cols; ++k) store_el(out, out_dt, r * cols + k, row[k]);
        }
        free(row);
    }
    return 0;
}

/* ------------------------------------------------------------------- qmm */

/* Row r of the weights in double: the dequantized values in T (exact_w = 0),
 * or scale*code + bias with scale and bias cast to T and no rounding after
 * (exact_w = 1). */
static void weight_row_f64(const uint32_t* wq, const void* scales, const void* biases, int sb_dt,
                           int T, int64_t r, int64_t K, int gs, int bits, int exact_w,
                           float* tmp, double* out) {
    if (!exact_w) {
        dequant_rows_f32(wq, scales, biases, sb_dt, T, r, K, gs, bits, tmp);
        for (int64_t k = 0; k < K; ++k) out[k] = (double)tmp[k];
        return;
    }
    const int64_t G = K / gs;
    const uint32_t* in = wq + r * (K * bits / 32);
    const uint32_t mask = (1u << bits) - 1u;
    for (int64_t g = 0; g < G; ++g) {
        const double sc = (double)round_to(T, load_el(scales, sb_dt, r * G + g));
        const double bi = (double)round_to(T, load_el(biases, sb_dt, r * G + g));
        for (int j = 0; j < gs; ++j) {
            const int64_t k = g * gs + j;
            const int64_t bit = k * bits;
            const int64_t w = bit >> 5;
            const int off = (int)(bit & 31);
            uint64_t win = in[w];
            if (off + bits > 32) win |= (uint64_t)in[w + 1] << 32;
            out[k] = sc * (double)(uint32_t)((win >> off) & mask) + bi;
        }
    }
}

/* transpose=1: y[m, rows] = x[m, cols] . W^T ; transpose=0: y[m, cols] = x[m, rows] . W.
 * T = promote(x_dt, sb_dt); x and the scales are cast to T, the weights are
 * weight_row_f64's values, the sum runs in double and is cast to y_dt. */
int rqo_qmm(const void* x, int x_dt, const uint32_t* wq, const void* scales, const void* biases,
            int sb_dt, int64_t m, int64_t rows, int64_t cols, int gs, int bits, int transpose,
            void* y, int y_dt, int nthreads, int exact_w) {
    if (!valid_bits(bits) || !valid_gs(gs) || !valid_dt(x_dt) || !valid_dt(sb_dt) ||
        !valid_dt(y_dt))
        return -1;
    if (m < 0 || rows < 0 || cols <= 0 || cols % gs != 0) return -1;
    const int T = rqo_promote(x_dt, sb_dt);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    if (transpose) {
        const int64_t K = cols;
        float* xf = (float*)malloc(sizeof(float) * (size_t)(m * K + 1));
        for (int64_t i = 0; i < m * K; ++i) xf[i] = round_to(T, load_el(x, x_dt, i));
#pragma omp parallel
        {
            float* tmp = (float*)malloc(sizeof(float) * (size_t)K);
            double* wrow = (double*)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(static)
            for (int64_t r = 0; r < rows; ++r) {
                weight_row_f64(wq, scales, biases, sb_dt, T, r, K, gs, bits, exact_w, tmp, wrow);
                for (int64_t i = 0; i < m; ++i) {
                    const float* xr = xf + i * K;
                    double acc = 0.0;
                    for (int64_t k = 0; k < K; ++k) acc += (double)xr[k] * wrow[k];
                    store_el(y, y_dt, i * rows + r, (float)acc);
                }
            }
            free(wrow);
            free(tmp);
        }
        free(xf);
    } else {
        const int64_t K = cols, R = rows;
        float* xf = (float*)malloc(sizeof(float) * (size_t)(m * R + 1));
        for (int64_t i = 0; i < m * R; ++i) xf[i] = round_to(T, load_el(x, x_dt, i));
        double* acc = (double*)calloc((size_t)(m * K + 1), sizeof(double));
        /* Each thread owns a contiguous slice of output columns; it
         * dequantizes every row but writes only its slice. */
#pragma omp parallel
        {
            float* tmp = (float*)malloc(sizeof(float) * (size_t)K);
            double* wrow = (double*)malloc(sizeof(double) * (size_t)K);
            int nt = 1, tid = 0;
#ifdef _OPENMP
            nt = omp_get_num_threads();
            tid = omp_get_thread_num();
#endif
            int64_t ngroups = K / gs;
            int64_t g0 = ngroups * tid / nt, g1 = ngroups * (tid + 1) / nt;
            int64_t k0 = g0 * gs, k1 = g1 * gs;
            for (int64_t r = 0; r < R; ++r) {
                if (k1 > k0) {
                    /* dequantize the whole row: simple, the slice is what is used */
                    weight_row_f64(wq, scales, biases, sb_dt, T, r, K, gs, bits, exact_w, tmp,
                                   wrow);
                    for (int64_t i = 0; i < m; ++i) {
                        double xv = xf[i * R + r];
                        double* ar = acc + i * K;
                        for (int64_t k = k0; k < k1; ++k) ar[k] += xv * wrow[k];
                    }
                }
            }
            free(wrow);
            free(tmp);
        }
        for (int64_t i = 0; i < m * K; ++i) store_el(y, y_dt, i, (float)acc[i]);
        free(acc);
        free(xf);
    }
    return 0;
}

/* GEMV restatement used as the timed CPU baseline (transpose=1, bf16 x and
 * bf16 scales).  Same result as rqo_qmm but organised like MLX's CPU qmv:
 * per group, sum x*code and x, then apply scale and bias once.  Single
 * precision accumulation per group, double across groups. */
int rqo_qmv_bf16(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                 const uint16_t* biases, int64_t m, int64_t rows, int64_t cols, int gs, int bits,
                 uint16_t* y, int nthreads) {
    if (!valid_bits(bits) || !valid_gs(gs) || cols % gs != 0 || m < 1 || m > 64) return -1;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    const int64_t K = cols, G = cols / gs, wpr = cols * bits / 32;
    const uint32_t mask = (1u << bits) - 1u;
    float* xf = (float*)malloc(sizeof(float) * (size_t)(m * K));
    float* xs = (float*)malloc(sizeof(float) * (size_t)(m * G));
    for (int64_t i = 0; i < m * K; ++i) xf[i] = bf16_to_f32(x[i]);
    for (int64_t i = 0; i < m; ++i)
        for (int64_t g = 0; g < G; ++g) {
            float s = 0.f;
            for (int j = 0; j < gs; ++j) s += xf[i * K + g * gs + j];
            xs[i * G + g] = s;
        }
#pragma omp parallel
    {
        uint8_t* codes = (uint8_t*)malloc((size_t)K);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            const uint32_t* in = wq + r * wpr;
            for (int64_t k = 0; k < K; ++k) {
                int64_t bit = k * bits;
                int64_t w = bit >> 5;
                int off = (int)(bit & 31);
                uint64_t win = in[w];
                if (off + bits > 32) win |= (uint64_t)in[w + 1] << 32;
                codes[k] = (uint8_t)((win >> off) & mask);
            }
            for (int64_t i = 0; i < m; ++i) {
                double acc = 0.0;
                const float* xr = xf + i * K;
                for (int64_t g = 0; g < G; ++g) {
                    float dot = 0.f;
                    for (int j = 0; j < gs; ++j) dot += xr[g * gs + j] * (float)codes[g * gs + j];
                    float s = bf16_to_f32(scales[r * G + g]);
                    float b = bf16_to_f32(biases[r * G + g]);
                    acc += (double)s * dot + (double)b * xs[i * G + g];
                }
                y[i * rows + r] = f32_to_bf16((float)acc);
            }
        }
        free(codes);
    }
    free(xf);
    free(xs);
    return 0;
}

/* ------------------------------------------------------------ sb6 / K3
 *
 * rwkv-quant "sb6" tensors in the K3-interleaved layout that RwkvqLinear
 * holds (layout stated at rwkv_metal/lora/rwkvq_kernel.py:18-25, arithmetic
 * at rwkv_metal/lora/rwkvq_linear.py:140-175 and rwkvq_kernel.py:86-100).
 * Blocks are 32 codes of one row (gw_gs = 32, rwkvq_kernel.py:36):
 *   qblk[row, blk] : 16 bytes, byte j = code j (low nibble) | code j+16
 *                    (high nibble); xbits >= 1 adds a uint32 whose bit c is
 *                    bit 4 of code c; xbits == 2 one more for bit 5;
 *   qsqm[row, blk] : (qs uint8, qm int8);
 *   ddm[row, sblk] : (d, dm) float16, sblk = blk / gw_sb;
 *   scale = f16(qs * d), min = f16(qm * dm) (fp32 products rounded to f16),
 *   w = code * scale + min in fp32 (code * scale is exact: at most 6 + 11
 *   significant bits, so this is one rounding however it is evaluated).
 * The native repack (rwkvq_native.py:49-78) stores max(scale, 1e-8) as the
 * affine scale and min as the bias, fp32, group size 32; the dense
 * dequantize of the fused kernel (rwkvq_kernel.py:86-100) has no clamp. */
void rqo_sb6_codes(const uint8_t* qblk, int64_t rows, int64_t cols, int xbits, uint8_t* codes) {
    const int64_t nb = cols / 32, bb = 16 + 4 * xbits;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* q = qblk + (r * nb + b) * bb;
            uint8_t* c = codes + r * cols + b * 32;
            for (int j = 0; j < 16; ++j) {
                c[j] = q[j] & 0xF;
                c[j + 16] = q[j] >> 4;
            }
            for (int x = 0; x < xbits; ++x) {
                const uint32_t plane = (uint32_t)q[16 + 4 * x] | ((uint32_t)q[17 + 4 * x] << 8) |
                                       ((uint32_t)q[18 + 4 * x] << 16) | ((uint32_t)q[19 + 4 * x] << 24);
                for (int k = 0; k < 32; ++k) c[k] |= (uint8_t)(((plane >> k) & 1u) << (4 + x));
            }
        }
}

void rqo_sb6_scale_min(const uint8_t* qsqm, const uint16_t* ddm, int64_t rows, int64_t cols,
                       int gw_sb, int clamp, float* scale, float* mn) {
    const int64_t nb = cols / 32, nsb = nb / gw_sb;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const float qs = (float)qsqm[(r * nb + b) * 2];
            const float qm = (float)(int8_t)qsqm[(r * nb + b) * 2 + 1];
            const float d = f16_to_f32(ddm[(r * nsb + b / gw_sb) * 2]);
            const float dm = f16_to_f32(ddm[(r * nsb + b / gw_sb) * 2 + 1]);
            float sc = round_to(RQ_F16, qs * d);
            if (clamp && !(sc >= 1e-8f)) sc = 1e-8f;
            scale[r * nb + b] = sc;
            mn[r * nb + b] = round_to(RQ_F16, qm * dm);
        }
}

int rqo_sb6_dequantize(const uint8_t* qblk, const uint8_t* qsqm, const uint16_t* ddm,
                       int64_t rows, int64_t cols, int gw_sb, int xbits, float* out) {
    if (cols % 32 || xbits < 0 || xbits > 2 || gw_sb <= 0 || (cols / 32) % gw_sb) return -1;
    const int64_t nb = cols / 32;
    uint8_t* codes = (uint8_t*)malloc((size_t)(rows * cols));
    float* sc = (float*)malloc((size_t)(rows * nb) * sizeof(float));
    float* mn = (float*)malloc((size_t)(rows * nb) * sizeof(float));
    rqo_sb6_codes(qblk, rows, cols, xbits, codes);
    rqo_sb6_scale_min(qsqm, ddm, rows, cols, gw_sb, 0, sc, mn);
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t k = 0; k < cols; ++k) {
            const float p = (float)codes[r * cols + k] * sc[r * nb + k / 32];
            out[r * cols + k] = p + mn[r * nb + k / 32];
        }
    free(codes);
    free(sc);
    free(mn);
    return 0;
}

int rqo_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
