/*
 * oracle.c -- CPU restatement of unillm's Q4_0 / Q8_0 linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP kernels and
 * the timed CPU baseline.  The product never links or calls it.
 *
 * Each function names the reference code it follows.  The arithmetic of the
 * live path is in candle-core 0.8 (external, un-vendored); its GGML block
 * formats are restated from their published definition.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int oracle_block_elems(int qtype) {
    if (qtype == ORACLE_Q4_0 || qtype == ORACLE_Q5_0 || qtype == ORACLE_Q8_0) return 32;
    if (qtype == ORACLE_Q4_K || qtype == ORACLE_Q5_K || qtype == ORACLE_Q6_K) return 256;
    return 0;
}

size_t oracle_block_bytes(int qtype) {
    /* Q4_0: {f16 d; u8 qs[16]} = 18 B; Q8_0: {f16 d; i8 qs[32]} = 34 B.
     * (The reference's in-repo Q4_0Block is 32 B because of align(32),
     * crates/runtime/src/simd/quant/block.rs:27 -- not the GGUF stride.)
     * Q4_K: 2 + 2 + 12 + 128 = 144 B; Q6_K: 128 + 64 + 16 + 2 = 210 B (GGML
     * block_q4_K / block_q6_K; the in-repo Q4_KBlock, block.rs:100-110, has
     * the same size but a simplified scale packing, block.rs:124-139, and is
     * not what candle's Q4K reads).  Q5_K: 2 + 2 + 12 + 32 + 128 = 176 B (GGML
     * block_q5_K). */
    if (qtype == ORACLE_Q4_0) return 18;
    if (qtype == ORACLE_Q5_0) return 22; /* {f16 d; u8 qh[4]; u8 qs[16]} (GGML block_q5_0) */
    if (qtype == ORACLE_Q8_0) return 34;
    if (qtype == ORACLE_Q4_K) return 144;
    if (qtype == ORACLE_Q5_K) return 176;
    if (qtype == ORACLE_Q6_K) return 210;
    return 0;
}

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* binary16 -> binary32, exact for every code (half::f16::to_f32 semantics,
 * used by candle's BlockQ4_0/BlockQ8_0::to_float). */
float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0) {
        if (man == 0) return bits_f32(sign);
        /* subnormal: man * 2^-24, exact in f32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) return bits_f32(sign | 0x7F800000u | (man << 13));
    return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* binary32 -> binary16, round to nearest even (half::f16::from_f32 and
 * x86 F16C _cvtss_sh(.., 0), which GGML_FP32_TO_FP16 uses). */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                       /* inf or nan */
        if (ax == 0x7F800000u) return sign | 0x7C00u;
        return sign | 0x7E00u | (uint16_t)((ax >> 13) & 0x3FFu);
    }
    if (ax >= 0x477FF000u) return sign | 0x7C00u;  /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                        /* below 2^-14: subnormal or 0 */
        if (ax < 0x33000000u) return sign;         /* < 2^-25: rounds to 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;                 /* 14..24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return sign | (uint16_t)q;
    }
    uint32_t e = (ax >> 23) - 112u;                /* 1..30 */
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;  /* carries into exp */
    return sign | (uint16_t)q;
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* GGML quantize_row_q4_0_reference, as candle's BlockQ4_0::from_float restates
 * it (candle-core 0.8 quantized/k_quants.rs, external): d = max / -8 where max
 * is the signed element of largest magnitude; q = min(15, trunc(x/d + 8.5));
 * low nibble of qs[j] holds element j, high nibble element j + 16. */
static void quantize_block_q4_0(const float* x, uint8_t* out) {
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < 32; ++j) {
        float v = x[j];
        if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
    }
    const float d = max / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    wr16(out, oracle_f32_to_f16(d));
    for (int j = 0; j < 16; ++j) {
        const float x0 = x[j] * id;
        const float x1 = x[j + 16] * id;
        int q0 = (int)(int8_t)(x0 + 8.5f);
        int q1 = (int)(int8_t)(x1 + 8.5f);
        if (q0 > 15) q0 = 15;
        if (q1 > 15) q1 = 15;
        out[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
}

/* GGML quantize_row_q8_0_reference / candle BlockQ8_0::from_float:
 * d = amax / 127; q = round-half-away(x / d). */
static void quantize_block_q8_0(const float* x, uint8_t* out) {
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) {
        float a = fabsf(x[j]);
        if (a > amax) amax = a;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    wr16(out, oracle_f32_to_f16(d));
    for (int j = 0; j < 32; ++j) out[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

int oracle_quantize(int qtype, const float* w, int64_t n, int64_t k, uint8_t* blocks) {
    const size_t bb = oracle_block_bytes(qtype);
    if ((qtype != ORACLE_Q4_0 && qtype != ORACLE_Q8_0) || k % 32 || n < 0 || k < 0) return -1;
    const int64_t kb = k / 32;
    for (int64_t r = 0; r < n; ++r)
        for (int64_t b = 0; b < kb; ++b) {
            const float* src = w + r * k + b * 32;
            uint8_t* dst = blocks + (size_t)(r * kb + b) * bb;
            if (qtype == ORACLE_Q4_0) quantize_block_q4_0(src, dst);
            else quantize_block_q8_0(src, dst);
        }
    return 0;
}

/* BlockQ4_0::to_float / BlockQ8_0::to_float (candle, external), reached from
 * qtensor.dequantize at crates/runtime/src/weight_loader_core.rs:579.  The
 * products are exact in f32 (<= 8-bit integer times an 11-bit significand). */
/* GGML get_scale_min_k4: sub-block j's 6-bit scale and min.  j < 4: low six
 * bits of scales[j] and scales[j + 4]; j >= 4: low / high nibble of
 * scales[j + 4] plus the top two bits of scales[j - 4] / scales[j]. */
static void q4_k_scale_min(int j, const uint8_t* q, int* sc, int* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* GGML dequantize_row_q4_K, one 256-weight block (BlockQ4K::to_float in candle,
 * the type weight_loader_core.rs:481 maps as Q4K).  d * sc and dmin * m are
 * exact in f32 (11-bit significand times 6 bits); (d sc) q is exact too, so the
 * one rounding is the subtraction, the same with or without a fused multiply-add. */
static void dequant_q4_k(const uint8_t* blk, float* y) {
    const float d = oracle_f16_to_f32(rd16(blk));
    const float dmin = oracle_f16_to_f32(rd16(blk + 2));
    const uint8_t* scales = blk + 4;
    const uint8_t* q = blk + 16;
    for (int g = 0; g < 4; ++g) {
        int sc, m;
        q4_k_scale_min(2 * g, scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        q4_k_scale_min(2 * g + 1, scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = dmin * (float)m;
        for (int l = 0; l < 32; ++l) y[64 * g + l] = d1 * (float)(q[32 * g + l] & 0x0F) - m1;
        for (int l = 0; l < 32; ++l) y[64 * g + 32 + l] = d2 * (float)(q[32 * g + l] >> 4) - m2;
    }
}

/* GGML dequantize_row_q5_K, one 256-weight block (BlockQ5K::to_float in candle;
 * GGUF Q5_K_M files hold their projections in it): Q4_K's scales, mins and
 * nibbles plus a fifth bit per weight in qh[32].  Weight l of sub-block 2 g
 * (g = 0..3, l = 0..31) takes the low nibble of qs[32 g + l] and bit 2 g of
 * qh[l]; weight l of sub-block 2 g + 1 the high nibble and bit 2 g + 1.  As for
 * Q4_K, (d sc) q is exact in f32 (q < 32) and the subtraction rounds once. */
static void dequant_q5_k(const uint8_t* blk, float* y) {
    const float d = oracle_f16_to_f32(rd16(blk));
    const float dmin = oracle_f16_to_f32(rd16(blk + 2));
    const uint8_t* scales = blk + 4;
    const uint8_t* qh = blk + 16;
    const uint8_t* q = blk + 48;
    for (int g = 0; g < 4; ++g) {
        int sc, m;
        q4_k_scale_min(2 * g, scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        q4_k_scale_min(2 * g + 1, scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = dmin * (float)m;
        for (int l = 0; l < 32; ++l) {
            const int q1 = (q[32 * g + l] & 0x0F) | (((qh[l] >> (2 * g)) & 1) << 4);
            const int q2 = (q[32 * g + l] >> 4) | (((qh[l] >> (2 * g + 1)) & 1) << 4);
            y[64 * g + l] = d1 * (float)q1 - m1;
            y[64 * g + 32 + l] = d2 * (float)q2 - m2;
        }
    }
}

/* GGML dequantize_row_q6_K, one 256-weight block: two halves of 128 weights,
 * each from 64 bytes of ql, 32 of qh and 8 scales; weight l + 32 t of a half
 * (t = 0..3, l = 0..31) has q = (ql nibble) | (2 bits of qh[l]) << 4, scale
 * scales[l / 16 + 2 t].  Evaluated as GGML writes it, (d * sc) * (q - 32):
 * d * sc is exact, the second product rounds once. */
static void dequant_q6_k(const uint8_t* blk, float* y) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    const float d = oracle_f16_to_f32(rd16(blk + 208));
    for (int h = 0; h < 2; ++h) {
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = ((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = ((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l] = d * (float)sc[is] * (float)q1;
            y[l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
        y += 128;
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

static void dequant_block(int qtype, const uint8_t* blk, float* y) {
    if (qtype == ORACLE_Q4_K) {
        dequant_q4_k(blk, y);
        return;
    }
    if (qtype == ORACLE_Q5_K) {
        dequant_q5_k(blk, y);
        return;
    }
    if (qtype == ORACLE_Q6_K) {
        dequant_q6_k(blk, y);
        return;
    }
    const float d = oracle_f16_to_f32(rd16(blk));
    if (qtype == ORACLE_Q5_0) {
        /* GGML dequantize_row_q5_0: the fifth bit of element j is bit j of the
         * little-endian u32 qh; (q - 16) * d is exact in f32 */
        const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) |
                            ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
        const uint8_t* qs = blk + 6;
        for (int j = 0; j < 16; ++j) {
            const int x0 = ((qs[j] & 0x0F) | (((qh >> j) & 1) << 4)) - 16;
            const int x1 = ((qs[j] >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16;
            y[j] = (float)x0 * d;
            y[j + 16] = (float)x1 * d;
        }
        return;
    }
    const uint8_t* qs = blk + 2;
    if (qtype == ORACLE_Q4_0) {
        for (int j = 0; j < 16; ++j) {
            y[j] = (float)((int)(qs[j] & 0x0F) - 8) * d;
            y[j + 16] = (float)((int)(qs[j] >> 4) - 8) * d;
        }
    } else {
        for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)qs[j] * d;
    }
}

int oracle_dequant(int qtype, const uint8_t* blocks, int64_t n, int64_t k, float* out) {
    const size_t bb = oracle_block_bytes(qtype);
    const int be = oracle_block_elems(qtype);
    if (!bb || n < 0 || k < 0 || k % be) return -1;
    const int64_t kb = k / be;
    for (int64_t r = 0; r < n; ++r)
        for (int64_t b = 0; b < kb; ++b)
            dequant_block(qtype, blocks + (size_t)(r * kb + b) * bb, out + r * k + b * be);
    return 0;
}

/* The parity oracle: the f32-fallback semantics of quantized_matmul
 * (crates/runtime/src/models_v2/llama.rs:1193 -> ops_fn::matmul ->
 * CpuTensorOpsImpl::matmul, crates/runtime/src/tensor_core.rs:843-892):
 * y = x . dequant(W)^T, here accumulated in f64 so it is a reference for any
 * f32 summation order.  x is [m, k] row-major (the 3-D [B, T, K] case of
 * tensor_core.rs:857-871 reshapes to [B*T, K]), W is [n, k] blocks. */
int oracle_qmatmul_f64(int qtype, const uint8_t* blocks, const float* x,
                       int64_t m, int64_t n, int64_t k, double* y, int nthreads) {
    const size_t bb = oracle_block_bytes(qtype);
    const int be = oracle_block_elems(qtype);
    if (!bb || n < 0 || k < 0 || m < 0 || k % be) return -1;
    const int64_t kb = k / be;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        float* wrow = (float*)malloc(sizeof(float) * (size_t)(k ? k : 1));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t c = 0; c < n; ++c) {
            for (int64_t b = 0; b < kb; ++b)
                dequant_block(qtype, blocks + (size_t)(c * kb + b) * bb, wrow + b * be);
            for (int64_t r = 0; r < m; ++r) {
                const float* xr = x + r * k;
                double acc = 0.0;
                for (int64_t i = 0; i < k; ++i) acc += (double)xr[i] * (double)wrow[i];
                y[r * n + c] = acc;
            }
        }
        free(wrow);
    }
    return 0;
}

/* ---- candle CPU QMatMul semantics (the timing baseline) -------------------
 * QMatMul::forward -> QTensor CustomOp1 cpu_fwd -> k_quants::matmul
 * (candle-core 0.8, external; called at llama.rs:1188, 1329, 399):
 *   1. each activation row is quantized to Q8_0 (VecDotType of Q4_0 and Q8_0);
 *   2. for each row, a rayon parallel-for over the N output columns
 *      (with_min_len 128, with_max_len 512) runs vec_dot over K/32 blocks:
 *      integer block dot, then sumf += isum * f32(d_w) * f32(d_x).
 * Restated with OpenMP dynamic chunks of 256 columns. */
static float vec_dot_q4_0_q8_0(const uint8_t* w, const uint8_t* xq, int64_t kb) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < kb; ++b, w += 18, xq += 34) {
        const uint8_t* qs = w + 2;
        const int8_t* ys = (const int8_t*)(xq + 2);
        int isum = 0;
        for (int j = 0; j < 16; ++j) {
            isum += ((int)(qs[j] & 0x0F) - 8) * ys[j];
            isum += ((int)(qs[j] >> 4) - 8) * ys[j + 16];
        }
        sumf += (float)isum * oracle_f16_to_f32(rd16(w)) * oracle_f16_to_f32(rd16(xq));
    }
    return sumf;
}

static float vec_dot_q8_0_q8_0(const uint8_t* w, const uint8_t* xq, int64_t kb) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < kb; ++b, w += 34, xq += 34) {
        const int8_t* qs = (const int8_t*)(w + 2);
        const int8_t* ys = (const int8_t*)(xq + 2);
        int isum = 0;
        for (int j = 0; j < 32; ++j) isum += qs[j] * ys[j];
        sumf += (float)isum * oracle_f16_to_f32(rd16(w)) * oracle_f16_to_f32(rd16(xq));
    }
    return sumf;
}

int oracle_candle_qmatmul(int qtype, const uint8_t* blocks, const float* x,
                          int64_t m, int64_t n, int64_t k, float* y, int nthreads) {
    const size_t bb = oracle_block_bytes(qtype);
    if ((qtype != ORACLE_Q4_0 && qtype != ORACLE_Q8_0) || k % 32 || n < 0 || k < 0 || m < 0)
        return -1;
    const int64_t kb = k / 32;
    uint8_t* xq = (uint8_t*)malloc((size_t)(m * kb * 34) + 1);
    if (!xq) return -2;
    oracle_quantize(ORACLE_Q8_0, x, m, k, xq);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
    for (int64_t r = 0; r < m; ++r) {
        const uint8_t* xr = xq + (size_t)(r * kb * 34);
        float* yr = y + r * n;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 256)
#endif
        for (int64_t c = 0; c < n; ++c) {
            const uint8_t* wc = blocks + (size_t)(c * kb) * bb;
            yr[c] = qtype == ORACLE_Q4_0 ? vec_dot_q4_0_q8_0(wc, xr, kb)
                                         : vec_dot_q8_0_q8_0(wc, xr, kb);
        }
    }
    free(xq);
    return 0;
}

/* ---- synthetic inputs ------------------------------------------------------ */
static inline uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void oracle_fill_normal(float* out, int64_t count, uint64_t seed, double mean, double std) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < count; i += 2) {
        double u1 = ((double)(splitmix64(&s) >> 11) + 0.5) * 0x1.0p-53;
        double u2 = ((double)(splitmix64(&s) >> 11) + 0.5) * 0x1.0p-53;
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + std * r * cos(two_pi * u2));
        if (i + 1 < count) out[i + 1] = (float)(mean + std * r * sin(two_pi * u2));
    }
}

/* ---- decode attention (see oracle.h) --------------------------------------------------- */
int oracle_attention_decode(const float* qkv, int64_t m, int64_t n_heads, int64_t n_kv_heads,
                            int64_t head_dim, float rope_theta, float* k_cache, float* v_cache,
                            int64_t max_seq, int64_t len, double* out) {
    if (m < 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || head_dim <= 0 ||
        head_dim % 2 || len < 0 || len + m > max_seq)
        return -1;
    const int64_t H = n_heads, KVH = n_kv_heads, D = head_dim, half = D / 2;
    const int64_t row = (H + 2 * KVH) * D, groups = H / KVH;
    /* inv_freq and the angles in f32, as apply_rope_with_offset builds them */
    float* inv = (float*)malloc(sizeof(float) * (size_t)half);
    for (int64_t i = 0; i < half; ++i) inv[i] = 1.0f / powf(rope_theta, (float)(2 * i) / (float)D);
    double* q = (double*)malloc(sizeof(double) * (size_t)(m * H * D));
    for (int64_t t = 0; t < m; ++t) {
        const float pos = (float)(len + t);
        const float* r = qkv + t * row;
        for (int64_t h = 0; h < H + KVH; ++h) {  /* q heads, then k heads */
            const float* x = r + h * D;
            for (int64_t i = 0; i < half; ++i) {
                const float ang = pos * inv[i];
                const double c = cos((double)ang), sn = sin((double)ang);
                const double a = x[i], b = x[i + half];
                const double r1 = a * c - b * sn, r2 = a * sn + b * c;
                if (h < H) {
                    q[(t * H + h) * D + i] = r1;
                    q[(t * H + h) * D + i + half] = r2;
                } else {
                    float* kc = k_cache + ((h - H) * max_seq + len + t) * D;
                    kc[i] = (float)r1;
                    kc[i + half] = (float)r2;
                }
            }
        }
        for (int64_t g = 0; g < KVH; ++g)  /* v: no rotation */
            memcpy(v_cache + (g * max_seq + len + t) * D, r + (H + KVH + g) * D,
                   sizeof(float) * (size_t)D);
    }
    /* LlamaAttention::new keeps 1 / sqrt(hd) in f32 (llama.rs:890); scores are scaled by it */
    const double scale = (double)(1.0f / sqrtf((float)D));
    double* sc = (double*)malloc(sizeof(double) * (size_t)(len + m));
    for (int64_t t = 0; t < m; ++t)
        for (int64_t h = 0; h < H; ++h) {
            const int64_t g = h / groups, n = len + t + 1;  /* causal: positions 0 .. len + t */
            const double* qh = q + (t * H + h) * D;
            double mx = -INFINITY;
            for (int64_t j = 0; j < n; ++j) {
                const float* kj = k_cache + (g * max_seq + j) * D;
                double s = 0.0;
                for (int64_t i = 0; i < D; ++i) s += qh[i] * (double)kj[i];
                sc[j] = s * scale;
                if (sc[j] > mx) mx = sc[j];
            }
            double z = 0.0;
            for (int64_t j = 0; j < n; ++j) z += (sc[j] = exp(sc[j] - mx));
            double* o = out + (t * H + h) * D;
            for (int64_t i = 0; i < D; ++i) o[i] = 0.0;
            for (int64_t j = 0; j < n; ++j) {
                const float* vj = v_cache + (g * max_seq + j) * D;
                const double p = sc[j] / z;
                for (int64_t i = 0; i < D; ++i) o[i] += p * (double)vj[i];
            }
        }
    free(sc);
    free(q);
    free(inv);
    return 0;
}
