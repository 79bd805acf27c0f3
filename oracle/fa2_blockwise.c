/*
 * CPU restatement of the reference's blockwise FlashAttention-2 forward.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ as a checker and never by the
 * product path.
 *
 * Follows Dell710000/ascend-rsfa ascend_rsfa/flash_attention_forward.py step
 * by step, including where it rounds:
 *   non-causal (_attn_fwd STAGE 1 -> _attn_fwd_inner STAGE 3, 369-404, 163-226):
 *     m = -inf, l = 1, acc = 0                                  (370-372)
 *     per BLOCK_N tile: qk = q.k^T (fp32); qk *= scale           (188, 199)
 *       m_ij = max(m, rowmax(qk)), NaN-propagating                (200-203)
 *       p = exp(qk - m_ij); p16 = (input dtype) p                (204-211)
 *       l = l * exp(m - m_ij) + rowsum(p)   (unrounded p)         (217-219)
 *       acc = acc * alpha + p16 . v                               (221-223)
 *     M = m + ln(l); O = (dtype)(acc / l)                         (400-404)
 *   causal (_run_causal_split, 493-541):
 *     prefix  (STAGE 4, 338-353 + _attn_fwd_split_inner STAGE 1, 408-489):
 *       keys [0, m*BM) in tiles of max(BM, BN), FA4 skip rule with
 *       threshold 0 (466-487); state (l, m) fp32; O = (dtype) acc, unnormalised
 *     diagonal (STAGE 5, 354-368 + split_inner STAGE 2):
 *       reload l, m, acc = (float) O; keys [m*BM, min((m+1)*BM, N)) in tiles of
 *       BN with the additive -1e6 mask where key > query (438-442);
 *       O = (dtype)(acc / l)
 *   small kernels (_attn_fwd_small / _small_causal, 26-159): one-tile softmax
 *   with an explicit division (small_head below), dispatched as at 564-581.
 * Dot products accumulate in float over the fp16/bf16 inputs, as the cube unit
 * does.  Shapes need N divisible by BM and BN, as in the reference.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float bits_to_f32(uint32_t x) {
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static uint32_t f32_to_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    return x;
}

/* IEEE binary16 <-> binary32, round to nearest even */
float rsfa_oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ff;
    if (exp == 0) {
        if (mant == 0) return bits_to_f32(sign);
        /* subnormal: mant * 2^-24 */
        float v = (float)mant * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) return bits_to_f32(sign | 0x7f800000u | (mant << 13));
    return bits_to_f32(sign | ((exp + 112) << 23) | (mant << 13));
}

uint16_t rsfa_oracle_f32_to_f16(float f) {
    uint32_t x = f32_to_bits(f);
    uint32_t sign = (x >> 16) & 0x8000;
    uint32_t exp = (x >> 23) & 0xff;
    uint32_t mant = x & 0x7fffff;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00 | (mant ? 0x200 : 0));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = mant | 0x800000u;
        int shift = 14 - e;
        uint32_t hm = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = mant >> 13;
    uint32_t rem = mant & 0x1fff;
    uint32_t h = sign | ((uint32_t)e << 10) | hm;
    if (rem > 0x1000 || (rem == 0x1000 && (hm & 1))) h++;
    return (uint16_t)h;
}

float rsfa_oracle_bf16_to_f32(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

uint16_t rsfa_oracle_f32_to_bf16(float f) {
    uint32_t x = f32_to_bits(f);
    if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x7fffffu)) return (uint16_t)((x >> 16) | 0x40);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

typedef struct {
    int bf16;
} dtype_ctx;

static float to_f32(const dtype_ctx* c, uint16_t h) {
    return c->bf16 ? rsfa_oracle_bf16_to_f32(h) : rsfa_oracle_f16_to_f32(h);
}

static uint16_t to_dt(const dtype_ctx* c, float f) {
    return c->bf16 ? rsfa_oracle_f32_to_bf16(f) : rsfa_oracle_f32_to_f16(f);
}

static float round_dt(const dtype_ctx* c, float f) { return to_f32(c, to_dt(c, f)); }

/* NaN-propagating max (tl.PropagateNan.ALL) */
static float max_nan(float a, float b) {
    if (isnan(a) || isnan(b)) return NAN;
    return a > b ? a : b;
}

/*
 * One KV loop over keys [lo, hi) for query rows [r0, r0 + bm) of one head.
 * stage 3: full range, plain update (_attn_fwd_inner)
 * stage 1: prefix, FA4 skip rule (_attn_fwd_split_inner STAGE 1)
 * stage 2: diagonal, mask + FA4 skip rule (_attn_fwd_split_inner STAGE 2)
 */
static void kv_loop(const dtype_ctx* c, const float* q, const float* k, const float* v, int d, int r0, int bm,
                    int lo, int hi, int bn, float scale, int stage, float* m_i, float* l_i, float* acc) {
    float* qk = (float*)malloc(sizeof(float) * (size_t)bm * bn);
    float* p16 = (float*)malloc(sizeof(float) * (size_t)bm * bn);
    for (int start = lo; start < hi; start += bn) {
        for (int i = 0; i < bm; ++i)
            for (int j = 0; j < bn; ++j) {
                const float* qr = q + (size_t)(r0 + i) * d;
                const float* kr = k + (size_t)(start + j) * d;
                float s = 0.0f;
                for (int t = 0; t < d; ++t) s += qr[t] * kr[t];
                s *= scale;
                if (stage == 2) s += ((r0 + i) >= (start + j)) ? 0.0f : -1.0e6f;
                qk[(size_t)i * bn + j] = s;
            }
        for (int i = 0; i < bm; ++i) {
            float rmax = qk[(size_t)i * bn];
            for (int j = 1; j < bn; ++j)
                rmax = stage == 2 ? fmaxf(rmax, qk[(size_t)i * bn + j]) : max_nan(rmax, qk[(size_t)i * bn + j]);
            const float m_ij = stage == 2 ? fmaxf(m_i[i], rmax) : max_nan(m_i[i], rmax);
            float lsum = 0.0f;
            for (int j = 0; j < bn; ++j) {
                const float pj = expf(qk[(size_t)i * bn + j] - m_ij);
                lsum += pj;
                p16[(size_t)i * bn + j] = round_dt(c, pj);
            }
            float alpha;
            if (stage == 3) {
                alpha = expf(m_i[i] - m_ij);
                l_i[i] = l_i[i] * alpha + lsum;
            } else {
                const float delta = m_ij - m_i[i];
                const int need = delta > 0.0f;
                alpha = need ? expf(-delta) : 1.0f;
                l_i[i] = (need ? l_i[i] * alpha : l_i[i]) + lsum;
            }
            float* ar = acc + (size_t)i * d;
            for (int t = 0; t < d; ++t) {
                float pv = 0.0f;
                for (int j = 0; j < bn; ++j) pv += p16[(size_t)i * bn + j] * v[(size_t)(start + j) * d + t];
                ar[t] = ar[t] * alpha + pv;
            }
            m_i[i] = m_ij;
        }
    }
    free(qk);
    free(p16);
}

/*
 * _attn_fwd_small / _attn_fwd_small_causal (26-89, 92-159): one tile per head,
 * qk = q.k^T * scale [+ -1e6 above the diagonal]; p = exp(qk - rowmax);
 * p /= rowsum(p); o = (dtype)((dtype)p . v).
 */
static void small_head(const dtype_ctx* c, const float* q, const float* k, const float* v, uint16_t* o, int n,
                       int d, float scale, int causal) {
    float* p = (float*)malloc(sizeof(float) * (size_t)n);
    for (int i = 0; i < n; ++i) {
        float mx = -INFINITY;
        for (int j = 0; j < n; ++j) {
            float s = 0.0f;
            for (int t = 0; t < d; ++t) s += q[(size_t)i * d + t] * k[(size_t)j * d + t];
            s *= scale;
            if (causal) s += (i >= j) ? 0.0f : -1.0e6f;
            p[j] = s;
            mx = j == 0 ? s : max_nan(mx, s);
        }
        float sum = 0.0f;
        for (int j = 0; j < n; ++j) {
            p[j] = expf(p[j] - mx);
            sum += p[j];
        }
        for (int j = 0; j < n; ++j) p[j] = round_dt(c, p[j] / sum);
        for (int t = 0; t < d; ++t) {
            float acc = 0.0f;
            for (int j = 0; j < n; ++j) acc += p[j] * v[(size_t)j * d + t];
            o[(size_t)i * d + t] = to_dt(c, acc);
        }
    }
    free(p);
}

/*
 * q, k, v, o: contiguous [Z, H, N, D] in fp16 (bf16 = 0) or bf16 (bf16 = 1).
 * Dispatch as in _attention.forward (564-583): the small kernels for
 * non-causal N <= 128 and causal N <= 64 (D <= 128), else the tiled paths.
 * lse: optional [Z, H, N] (non-causal only, as in the reference).
 * Returns 0, or -1 for shapes the reference cannot run.
 */
int rsfa_oracle_fa2_forward(const uint16_t* q16, const uint16_t* k16, const uint16_t* v16, uint16_t* o16,
                            float* lse, int z, int h, int n, int d, float sm_scale, int causal, int bm, int bn,
                            int bf16) {
    const int small = d <= 128 && ((!causal && n <= 128) || (causal && n <= 64));
    if (!small && (bm <= 0 || bn <= 0 || n % bm != 0 || n % bn != 0)) return -1;
    if (!small && causal && bn > bm) return -1;
    const int bn_prefix = bm > bn ? bm : bn;
    if (!small && causal && bm % bn_prefix != 0) return -1;
    dtype_ctx c = {bf16};
    const size_t hs = (size_t)n * d;
    float* q = (float*)malloc(sizeof(float) * hs);
    float* k = (float*)malloc(sizeof(float) * hs);
    float* v = (float*)malloc(sizeof(float) * hs);
    const int bmx = bm > 0 ? bm : 1;
    float* m_i = (float*)malloc(sizeof(float) * (size_t)bmx);
    float* l_i = (float*)malloc(sizeof(float) * (size_t)bmx);
    float* acc = (float*)malloc(sizeof(float) * (size_t)bmx * d);
    for (int zh = 0; zh < z * h; ++zh) {
        const size_t base = (size_t)zh * hs;
        for (size_t i = 0; i < hs; ++i) {
            q[i] = to_f32(&c, q16[base + i]);
            k[i] = to_f32(&c, k16[base + i]);
            v[i] = to_f32(&c, v16[base + i]);
        }
        if (small) {
            small_head(&c, q, k, v, o16 + base, n, d, sm_scale, causal);
            continue;
        }
        for (int mb = 0; mb < n / bm; ++mb) {
            const int r0 = mb * bm;
            for (int i = 0; i < bm; ++i) {
                m_i[i] = -INFINITY;
                l_i[i] = 1.0f;
            }
            memset(acc, 0, sizeof(float) * (size_t)bm * d);
            if (!causal) {
                kv_loop(&c, q, k, v, d, r0, bm, 0, n, bn, sm_scale, 3, m_i, l_i, acc);
                for (int i = 0; i < bm; ++i) {
                    if (lse) lse[(size_t)zh * n + r0 + i] = m_i[i] + logf(l_i[i]);
                    for (int t = 0; t < d; ++t)
                        o16[base + (size_t)(r0 + i) * d + t] = to_dt(&c, acc[(size_t)i * d + t] / l_i[i]);
                }
            } else {
                /* prefix launch: stores l, m and the unnormalised acc in the output dtype */
                kv_loop(&c, q, k, v, d, r0, bm, 0, r0, bn_prefix, sm_scale, 1, m_i, l_i, acc);
                for (size_t i = 0; i < (size_t)bm * d; ++i) acc[i] = round_dt(&c, acc[i]);
                /* diagonal launch */
                const int hi = (r0 + bm) < n ? (r0 + bm) : n;
                kv_loop(&c, q, k, v, d, r0, bm, r0, hi, bn, sm_scale, 2, m_i, l_i, acc);
                for (int i = 0; i < bm; ++i)
                    for (int t = 0; t < d; ++t)
                        o16[base + (size_t)(r0 + i) * d + t] = to_dt(&c, acc[(size_t)i * d + t] / l_i[i]);
            }
        }
    }
    free(q);
    free(k);
    free(v);
    free(m_i);
    free(l_i);
    free(acc);
    return 0;
}
