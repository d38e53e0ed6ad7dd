/*
 * attn_oracle.c -- CPU restatement of the reference attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the checker
 * (or the timed CPU baseline).  The product library (libattn_mi355x.so) never
 * links, loads or calls anything in this directory.
 *
 * Reference: MarcVivas/llm-inference.  Every function cites the reference
 * file:line whose arithmetic it restates.  All fp16 values are IEEE binary16
 * bit patterns held in uint16_t.  Build with -ffp-contract=off (see Makefile)
 * so that every fp32 product and sum is rounded exactly once, as written.
 *
 * How each function is pinned (what would catch a plausible mistake):
 *   orc_f32_to_f16 / orc_f16_to_f32   exhaustive/edge comparison with numpy's
 *                                     float16 casts (tests/test_oracle.py).
 *   orc_rope_tables                   position 0 is exactly (1, 0); values vs
 *                                     fp64 cos/sin within one fp16 ulp; the
 *                                     theta=5e6 SmolLM3 frequencies.
 *   orc_rope_store_kv                 closed form: position 0 leaves Q/K
 *                                     bit-identical; rotation by (pi/2) swaps
 *                                     halves; norm preserved within fp16
 *                                     rounding; NoPE/V copies bit-exact;
 *                                     untouched rows/sources bit-exact.
 *   orc_attention                     the reference's own Flash-Decode
 *                                     known-answer inputs (closed form,
 *                                     test_causal_attention.cpp:152-228) against
 *                                     an independent numpy fp64 softmax
 *                                     (tests/golden/make_golden.py); torch
 *                                     scaled_dot_product_attention (a library)
 *                                     on random causal GQA inputs; invariants
 *                                     (L=1 -> V[0]; constant K -> mean V; row t
 *                                     independent of rows > t).
 *   orc_attention_chunked             equals orc_attention within fp32 error for
 *                                     every chunk size (an unscaled merge fails).
 *   orc_gemv, orc_gemm                numpy's float64 matrix-vector product (a
 *                                     library routine) on non-square shapes (a
 *                                     transposed W fails); identity rows copy x
 *                                     exactly; the reference's own
 *                                     test_matrix_vec_mul.cpp inputs (closed
 *                                     form) within its tolerance of fp64.
 *   orc_gemv_beta                     beta = 0 equals orc_gemv bit for bit;
 *                                     W = 0 leaves y (beta = 1) / gives
 *                                     fp16(beta y); a hand-worked case whose
 *                                     result differs when the product is
 *                                     rounded to fp16 before the residual is
 *                                     added (a double rounding fails).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- fp16 --- */

/* Round-to-nearest-even float -> binary16, the rounding of __float2half used
 * throughout the reference (e.g. rope.hip.cpp:56-57, causal_attention.hip.cpp:371). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7fffffffu;
    if (absx > 0x7f800000u) return (uint16_t)(sign | 0x7e00u); /* NaN */
    if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
    if (absx < 0x38800000u) {
        /* subnormal half (or zero): value = m * 2^-24 */
        if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        uint32_t e = absx >> 23;
        uint32_t m = (absx & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* 14..24 */
        uint32_t r = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t e = (absx >> 23) - 112u; /* rebias 127 -> 15 */
    uint32_t m = absx & 0x7fffffu;
    uint32_t r = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            float v = (float)m * (1.0f / 16777216.0f); /* m * 2^-24, exact */
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void orc_f32_to_f16_array(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_f32_to_f16(src[i]);
}

void orc_f16_to_f32_array(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_f16_to_f32(src[i]);
}

/* ---------------------------------------------------------------- RoPE --- */

/* rope_cache.hpp:48-60 (compute_inverse_frequencies) and :62-76
 * (fill_host_tables): inv_freq[i] = 1 / powf(theta, 2i/D) in fp32;
 * angle = float(pos) * inv_freq[i]; cos/sin evaluated in fp32 and rounded to
 * fp16.  Tables are [S][D/2]. */
void orc_rope_tables(uint16_t* cos_out, uint16_t* sin_out, size_t max_seq_len,
                     size_t head_dim, float theta) {
    size_t half = head_dim / 2;
    for (size_t i = 0; i < half; ++i) {
        float exponent = (float)(2 * i) / (float)head_dim;
        float inv = 1.0f / powf(theta, exponent);
        for (size_t pos = 0; pos < max_seq_len; ++pos) {
            float angle = (float)pos * inv;
            cos_out[pos * half + i] = orc_f32_to_f16(cosf(angle));
            sin_out[pos * half + i] = orc_f32_to_f16(sinf(angle));
        }
    }
}

/* rope.hip.cpp:44-58 (rotate_pair): x0 = x[i], x1 = x[i + D/2];
 * out0 = fp16(x0*c - x1*s), out1 = fp16(x1*c + x0*s), fp32 arithmetic with
 * each product rounded (no fused multiply-add). */
static void rotate_head(const uint16_t* src, uint16_t* dst, const uint16_t* cosr,
                        const uint16_t* sinr, size_t half) {
    for (size_t i = 0; i < half; ++i) {
        float c = orc_f16_to_f32(cosr[i]);
        float s = orc_f16_to_f32(sinr[i]);
        float x0 = orc_f16_to_f32(src[i]);
        float x1 = orc_f16_to_f32(src[i + half]);
        float a = x0 * c;
        float b = x1 * s;
        float d = x1 * c;
        float e = x0 * s;
        dst[i] = orc_f32_to_f16(a - b);
        dst[i + half] = orc_f32_to_f16(d + e);
    }
}

/* rope.hip.cpp:61-134 (rope_and_store_kv), :9-42 (copy_to_kv_cache) and the
 * launcher :138-196.  Token t uses table row start_pos + t.
 *   apply != 0: Q head h of token t rotated in place at q + t*q_stride + h*D;
 *               K rotated from k + t*k_stride + h*D into
 *               k_cache + (start_pos+t)*Hkv*D + h*D (K source unchanged);
 *               V copied to the same cache index of v_cache.
 *               k_cache == NULL: K rotated in place, V untouched (launch_rope,
 *               rope.hip.cpp:120-125, :198-205).
 *   apply == 0: K and V copied into the caches; Q untouched.
 * V is read with k_stride (rope.hip.cpp:109, :131; copy_to_kv_cache :33). */
void orc_rope_store_kv(uint16_t* q, uint16_t* k, const uint16_t* v,
                       uint16_t* k_cache, uint16_t* v_cache,
                       const uint16_t* cos_t, const uint16_t* sin_t,
                       size_t seq_len, size_t num_heads, size_t num_kv_heads,
                       size_t head_dim, size_t q_stride, size_t k_stride,
                       size_t start_pos, int apply_rotation) {
    size_t half = head_dim / 2;
    size_t kv_dim = num_kv_heads * head_dim;
    uint16_t tmp[4096];
    for (size_t t = 0; t < seq_len; ++t) {
        const uint16_t* cr = cos_t + (start_pos + t) * half;
        const uint16_t* sr = sin_t + (start_pos + t) * half;
        if (apply_rotation) {
            for (size_t h = 0; h < num_heads; ++h) {
                uint16_t* x = q + t * q_stride + h * head_dim;
                rotate_head(x, tmp, cr, sr, half);
                memcpy(x, tmp, 2 * half * sizeof(uint16_t));
            }
        }
        for (size_t h = 0; h < num_kv_heads; ++h) {
            uint16_t* ks = k + t * k_stride + h * head_dim;
            const uint16_t* vs = v ? v + t * k_stride + h * head_dim : NULL;
            size_t dst = (start_pos + t) * kv_dim + h * head_dim;
            if (apply_rotation) {
                rotate_head(ks, tmp, cr, sr, half);
                if (k_cache == NULL) {
                    memcpy(ks, tmp, 2 * half * sizeof(uint16_t));
                } else {
                    memcpy(k_cache + dst, tmp, 2 * half * sizeof(uint16_t));
                    memcpy(v_cache + dst, vs, 2 * half * sizeof(uint16_t));
                }
            } else {
                memcpy(k_cache + dst, ks, head_dim * sizeof(uint16_t));
                memcpy(v_cache + dst, vs, head_dim * sizeof(uint16_t));
            }
        }
    }
}

/* ----------------------------------------------------------- attention --- */

/* Grouped-query causal attention, fp64 softmax.
 * Restates causal_attention.hip.cpp:148-183 (score = q.k / sqrt(D), key j
 * masked when j >= kv_len or j > q_pos0 + t), :210-268 and :361-372 (softmax
 * normalisation), the GQA head map kv_head = h / (Hq/Hkv) (:293, :510), and
 * python/reference.py:79-92 (repeat_interleave + SDPA is_causal).  The
 * arithmetic follows the reference's own fp64 CPU oracle,
 * tests/test_causal_attention.cpp:176-196 (double dot, exp(score - max),
 * numerator/denominator, then float -> fp16).
 *   Q row t, head h at q[t*q_stride + h*D]; K/V row j, kv head g at
 *   k[j*kv_stride + g*D]; out is packed [Nq][Hq][D].
 *   causal == 0: every key j < kv_len is visible (decode, Q1 in the survey:
 *   causal_attention.hip.cpp:943).
 * out16 (fp16 bits) and/or out32 (the exact value before rounding) may be NULL.
 * rows: optional list of n_rows query rows to evaluate (NULL = all Nq rows);
 * output row r of a list goes to out[r]. */
int orc_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                  uint16_t* out16, float* out32, size_t nq, size_t num_heads,
                  size_t num_kv_heads, size_t head_dim, size_t q_stride,
                  size_t kv_stride, size_t kv_len, size_t q_pos0, int causal,
                  const int64_t* rows, size_t n_rows) {
    if (num_kv_heads == 0 || num_heads % num_kv_heads != 0 || head_dim > 1024) return -1;
    size_t group = num_heads / num_kv_heads;
    double qd[1024];
    size_t count = rows ? n_rows : nq;
    for (size_t r = 0; r < count; ++r) {
        size_t t = rows ? (size_t)rows[r] : r;
        size_t end = kv_len;
        if (causal && q_pos0 + t + 1 < end) end = q_pos0 + t + 1;
        for (size_t h = 0; h < num_heads; ++h) {
            size_t g = h / group;
            const uint16_t* qrow = q + t * q_stride + h * head_dim;
            for (size_t c = 0; c < head_dim; ++c) qd[c] = (double)orc_f16_to_f32(qrow[c]);
            double inv_sqrt = 1.0 / sqrt((double)head_dim);
            double maximum = -INFINITY;
            /* first pass: maximum */
            for (size_t j = 0; j < end; ++j) {
                const uint16_t* kr = k + j * kv_stride + g * head_dim;
                double dot = 0.0;
                for (size_t c = 0; c < head_dim; ++c) dot += qd[c] * (double)orc_f16_to_f32(kr[c]);
                double s = dot * inv_sqrt;
                if (s > maximum) maximum = s;
            }
            double den = 0.0;
            double num[1024];
            for (size_t c = 0; c < head_dim; ++c) num[c] = 0.0;
            for (size_t j = 0; j < end; ++j) {
                const uint16_t* kr = k + j * kv_stride + g * head_dim;
                const uint16_t* vr = v + j * kv_stride + g * head_dim;
                double dot = 0.0;
                for (size_t c = 0; c < head_dim; ++c) dot += qd[c] * (double)orc_f16_to_f32(kr[c]);
                double w = exp(dot * inv_sqrt - maximum);
                den += w;
                for (size_t c = 0; c < head_dim; ++c) num[c] += w * (double)orc_f16_to_f32(vr[c]);
            }
            size_t o = (r * num_heads + h) * head_dim;
            for (size_t c = 0; c < head_dim; ++c) {
                float val = end ? (float)(num[c] / den) : 0.0f;
                if (out32) out32[o + c] = val;
                if (out16) out16[o + c] = orc_f32_to_f16(val);
            }
        }
    }
    return 0;
}

/* Chunked single-query attention with a partial-softmax merge in fp32:
 * causal_attention.hip.cpp:619-716 (per chunk: max, exp(score - max), chunk
 * weight sum and unnormalised P.V in fp32) and :719-838 (merge: global max
 * M = max_c m_c, l = sum_c exp(m_c - M) l_c, out = sum_c exp(m_c - M) acc_c / l).
 * One query token, all kv_len keys visible.  out32 is [Hq][D]. */
int orc_attention_chunked(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                          float* out32, size_t num_heads, size_t num_kv_heads,
                          size_t head_dim, size_t kv_stride, size_t kv_len,
                          size_t chunk) {
    if (num_kv_heads == 0 || num_heads % num_kv_heads != 0 || head_dim > 1024 ||
        chunk == 0 || chunk > 4096 || kv_len == 0)
        return -1;
    size_t group = num_heads / num_kv_heads;
    float inv = (float)(1.0 / sqrt((double)head_dim));
    size_t nchunks = (kv_len + chunk - 1) / chunk;
    for (size_t h = 0; h < num_heads; ++h) {
        size_t g = h / group;
        const uint16_t* qrow = q + h * head_dim;
        float gmax = -INFINITY;
        /* pass over chunks to find the global max of the chunk maxima */
        for (size_t c = 0; c < nchunks; ++c) {
            size_t j1 = (c + 1) * chunk < kv_len ? (c + 1) * chunk : kv_len;
            for (size_t j = c * chunk; j < j1; ++j) {
                float dot = 0.0f;
                for (size_t d = 0; d < head_dim; ++d)
                    dot += orc_f16_to_f32(qrow[d]) *
                           orc_f16_to_f32(k[j * kv_stride + g * head_dim + d]);
                float s = dot * inv;
                if (s > gmax) gmax = s;
            }
        }
        float lsum = 0.0f;
        float acc_out[1024];
        for (size_t d = 0; d < head_dim; ++d) acc_out[d] = 0.0f;
        for (size_t c = 0; c < nchunks; ++c) {
            size_t j0 = c * chunk;
            size_t j1 = (c + 1) * chunk < kv_len ? (c + 1) * chunk : kv_len;
            float sc[4096];
            float m = -INFINITY;
            for (size_t j = j0; j < j1; ++j) {
                float dot = 0.0f;
                for (size_t d = 0; d < head_dim; ++d)
                    dot += orc_f16_to_f32(qrow[d]) *
                           orc_f16_to_f32(k[j * kv_stride + g * head_dim + d]);
                sc[j - j0] = dot * inv;
                if (sc[j - j0] > m) m = sc[j - j0];
            }
            float l = 0.0f;
            float acc[1024];
            for (size_t d = 0; d < head_dim; ++d) acc[d] = 0.0f;
            for (size_t j = j0; j < j1; ++j) {
                float w = expf(sc[j - j0] - m);
                l += w;
                for (size_t d = 0; d < head_dim; ++d)
                    acc[d] += w * orc_f16_to_f32(v[j * kv_stride + g * head_dim + d]);
            }
            float scale = expf(m - gmax);
            lsum += scale * l;
            for (size_t d = 0; d < head_dim; ++d) acc_out[d] += scale * acc[d];
        }
        for (size_t d = 0; d < head_dim; ++d) out32[h * head_dim + d] = acc_out[d] / lsum;
    }
    return 0;
}

/* ------------------------------------------------------------ KV cache --- */

/* kv_cache.hpp:20-34, :76-82: one buffer for all layers; layer l starts at
 * l * 2*S*Hkv*D elements; K first, then V at + S*Hkv*D; row t of kv head h at
 * t*Hkv*D + h*D inside each. */
size_t orc_kv_k_offset(size_t layer, size_t max_seq_len, size_t num_kv_heads, size_t head_dim) {
    return layer * 2 * num_kv_heads * head_dim * max_seq_len;
}

size_t orc_kv_v_offset(size_t layer, size_t max_seq_len, size_t num_kv_heads, size_t head_dim) {
    return orc_kv_k_offset(layer, max_seq_len, num_kv_heads, head_dim) +
           max_seq_len * num_kv_heads * head_dim;
}

/* kv_cache.hpp:71-73 */
size_t orc_kv_total_bytes(size_t num_layers, size_t max_seq_len, size_t num_kv_heads,
                          size_t head_dim) {
    return 2 * num_kv_heads * head_dim * max_seq_len * 2 * num_layers;
}

/* -------------------------------------------------- reference KAT inputs --- */

/* tests/test_causal_attention.cpp:165-175: q[i] = fp16(2 sin(0.37 (i+1))),
 * k[t*stride + i] = fp16(3 cos(0.13 (t*kv_dim + i + 1))),
 * v[t*stride + i] = fp16(sin(0.19 (t*kv_dim + i + 3))), every other element of
 * the (len + 2) * stride K/V buffers = fp16(123). fp32 libm arithmetic. */
void orc_kat_inputs(uint16_t* q, uint16_t* k, uint16_t* v, size_t q_dim, size_t len,
                    size_t kv_dim, size_t stride) {
    for (size_t i = 0; i < q_dim; ++i) q[i] = orc_f32_to_f16(2.f * sinf((float)(i + 1) * .37f));
    uint16_t sentinel = orc_f32_to_f16(123.f);
    for (size_t i = 0; i < (len + 2) * stride; ++i) {
        k[i] = sentinel;
        v[i] = sentinel;
    }
    for (size_t t = 0; t < len; ++t)
        for (size_t i = 0; i < kv_dim; ++i) {
            k[t * stride + i] = orc_f32_to_f16(3.f * cosf((float)(t * kv_dim + i + 1) * .13f));
            v[t * stride + i] = orc_f32_to_f16(sinf((float)(t * kv_dim + i + 3) * .19f));
        }
}

/* ---------------------------------------------------------------- GEMV --- */

/* y[r] = fp16(sum_c W[r][c] * x[c]) for r < out_dim: the beta = 0 GEMV that
 * launch_qkv_decode runs (qkv_gemm.hip.cpp:107-116 ->
 * matrix_vec_mul.hip.cpp:79-172).  The reference accumulates fp32 products in
 * a thread- and lane-dependent order, then rounds the fp32 sum to fp16
 * (:150).  Here every product of two fp16 values is exact in fp64 and the sum
 * is carried in fp64, so this is the order-free value the reference's fp32
 * sum approximates; the fp64 sum is rounded to fp32, then to fp16 (RNE) as in
 * :150.  A GPU result can differ from it only by the fp32 summation error
 * around an fp16 rounding boundary (one fp16 ulp in rare elements). */
void orc_gemv(const uint16_t* w, const uint16_t* x, uint16_t* y, size_t out_dim, size_t in_dim) {
    for (size_t r = 0; r < out_dim; ++r) {
        const uint16_t* row = w + r * in_dim;
        double acc = 0.0;
        for (size_t c = 0; c < in_dim; ++c)
            acc += (double)orc_f16_to_f32(row[c]) * (double)orc_f16_to_f32(x[c]);
        y[r] = orc_f32_to_f16((float)acc);
    }
}

/* y = W x + beta * y, the residual form of the same GEMV
 * (matrix_vec_mul.hip.cpp:156-163; launch_attention_out_projection_decode,
 * attention_out_projection.hip.cpp:61-71, with beta = 1 on the engine's
 * residual stream, model_inference.hpp:390-397): the fp32 sum of W x (fp64
 * here, rounded to fp32 as orc_gemv does), plus the fp32 product beta * y[r]
 * when beta != 0, rounded once to fp16.  y is read and written in place. */
void orc_gemv_beta(const uint16_t* w, const uint16_t* x, uint16_t* y, size_t out_dim,
                   size_t in_dim, float beta) {
    for (size_t r = 0; r < out_dim; ++r) {
        const uint16_t* row = w + r * in_dim;
        double acc = 0.0;
        for (size_t c = 0; c < in_dim; ++c)
            acc += (double)orc_f16_to_f32(row[c]) * (double)orc_f16_to_f32(x[c]);
        float sum = (float)acc;
        if (beta != 0.0f) {
            const float res = beta * orc_f16_to_f32(y[r]);
            sum = sum + res;
        }
        y[r] = orc_f32_to_f16(sum);
    }
}

/* y[m][n] = fp16(sum_k x[m][k] * w[n][k]) for m < rows, n < out_dim: the
 * prefill QKV projection of launch_qkv_gemm (qkv_gemm.hip.cpp:7-105, rocBLAS
 * gemm_ex with fp32 compute and fp16 output), row by row as orc_gemv: exact
 * fp16 products, fp64 sum, rounded to fp32 then fp16. */
void orc_gemm(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t rows, size_t out_dim,
              size_t in_dim) {
    /* the same arithmetic as orc_gemv per row, with W and each x row widened
     * once instead of per product */
    double* wd = (double*)malloc(sizeof(double) * (out_dim * in_dim + in_dim + 1));
    if (!wd) {
        for (size_t m = 0; m < rows; ++m)
            orc_gemv(w, x + m * in_dim, y + m * out_dim, out_dim, in_dim);
        return;
    }
    double* xd = wd + out_dim * in_dim;
    for (size_t i = 0; i < out_dim * in_dim; ++i) wd[i] = (double)orc_f16_to_f32(w[i]);
    for (size_t m = 0; m < rows; ++m) {
        for (size_t c = 0; c < in_dim; ++c) xd[c] = (double)orc_f16_to_f32(x[m * in_dim + c]);
        for (size_t r = 0; r < out_dim; ++r) {
            const double* row = wd + r * in_dim;
            double acc = 0.0;
            for (size_t c = 0; c < in_dim; ++c) acc += row[c] * xd[c];
            y[m * out_dim + r] = orc_f32_to_f16((float)acc);
        }
    }
    free(wd);
}
