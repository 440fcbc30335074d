/*
 * nf4_oracle.c - CPU restatement of the AethelStream NF4 streamed-weight path.
 *
 * TEST INFRASTRUCTURE ONLY (see nf4_oracle.h for who may load it and how each
 * function is pinned).  Compiled with -O2 -fno-fast-math -ffp-contract=off so
 * that every fp32 operation is a single IEEE-754 correctly rounded operation,
 * as in the reference (Rust f32 and torch CPU fp32 both are).
 */
#include "nf4_oracle.h"

#include <math.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* shard_engine/src/nf4.rs:6-23 (same decimal literals as
 * shard_engine/python/pipeline/quantizer.py:5-10). */
static const float kCodes[16] = {
    -1.0f,        -0.6961928f, -0.52507305f, -0.3949175f,
    -0.28444138f, -0.18477343f, -0.09105004f, 0.0f,
    0.0795803f,   0.1609302f,  0.2461123f,   0.33791524f,
    0.44070983f,  0.562617f,   0.72295684f,  1.0f,
};

void or_codebook(float out[16]) { memcpy(out, kCodes, sizeof(kCodes)); }

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* binary32 -> binary16, IEEE round to nearest even (half 2.7.1
 * f16::from_f32 semantics, used at shard_engine/src/nf4.rs:78).  NaN keeps
 * its sign and becomes a quiet NaN carrying the top payload bits. */
uint16_t or_f32_to_f16(float x) {
    uint32_t u = f2u(x);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t e = (u >> 23) & 0xffu;
    uint32_t m = u & 0x7fffffu;
    if (e == 0xffu) {
        if (m == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (m >> 13));
    }
    int32_t he = (int32_t)e - 127 + 15;
    if (he >= 31) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
    if (he <= 0) {
        /* subnormal half (or zero): value = mant24 * 2^(e-150); half
         * subnormal unit is 2^-24, so shift right by (126 - e). */
        if (e == 0) return (uint16_t)sign; /* fp32 subnormals << 2^-24 */
        uint32_t mant = m | 0x800000u;
        int32_t shift = 126 - (int32_t)e; /* >= 14 */
        if (shift > 24) return (uint16_t)sign;
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q); /* q may carry into the exponent: ok */
    }
    uint32_t q = ((uint32_t)he << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u; /* may -> inf */
    return (uint16_t)(sign | q);
}

/* binary32 -> bfloat16, round to nearest even; NaN -> quiet NaN. */
uint16_t or_f32_to_bf16(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

float or_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        float v = (float)m * 0x1p-24f;
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e - 15 + 127) << 23) | (m << 13));
}

/* quantizer.py:40-41: distances = |n - code_i| in fp32, argmin over i with
 * the first minimum winning. */
uint8_t or_nf4_code_argmin(float n) {
    uint8_t best = 0;
    float bd = fabsf(n - kCodes[0]);
    for (int i = 1; i < 16; ++i) {
        float d = fabsf(n - kCodes[i]);
        if (d < bd) { bd = d; best = (uint8_t)i; }
    }
    return best;
}

/* Bracketing rule: j = last index with code_j <= n; choose between j and
 * j+1 by the same rounded distances, j on a tie.  Any other index is at least
 * one codebook gap (>= 0.0795) farther, far above one ulp of a value <= 2,
 * so it can never tie or win; or_check_bracket_exhaustive confirms it. */
uint8_t or_nf4_code_bracket(float n) {
    int j = 0;
    for (int i = 1; i < 16; ++i) j += (n >= kCodes[i]);
    if (j == 15) return 15;
    float dl = fabsf(n - kCodes[j]);
    float dr = fabsf(n - kCodes[j + 1]);
    return (uint8_t)(dr < dl ? j + 1 : j);
}

int64_t or_check_bracket_exhaustive(int nthreads) {
    /* Every fp32 bit pattern in [0, 1] and [-1, -0]. */
    const uint32_t one = 0x3f800000u;
    int64_t bad = 0;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
#pragma omp parallel for reduction(+ : bad) schedule(static, 1 << 16)
    for (int64_t b = 0; b <= (int64_t)one; ++b) {
        float p = u2f((uint32_t)b);
        float q = u2f((uint32_t)b | 0x80000000u);
        bad += or_nf4_code_argmin(p) != or_nf4_code_bracket(p);
        bad += or_nf4_code_argmin(q) != or_nf4_code_bracket(q);
    }
    return bad;
}

/* A candidate step form of the same rule: code(n) = #{k : n >= steps[k]}
 * for 15 ascending fp32 thresholds.  Returns how many fp32 n in [-1, 1]
 * (every bit pattern, both signs) get a different code from the 16-way
 * argmin of quantizer.py:40-41; 0 means the thresholds reproduce it. */
int64_t or_check_steps_exhaustive(const float *steps, int nthreads) {
    const uint32_t one = 0x3f800000u;
    int64_t bad = 0;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
#pragma omp parallel for reduction(+ : bad) schedule(static, 1 << 16)
    for (int64_t b = 0; b <= (int64_t)one; ++b) {
        const float p = u2f((uint32_t)b);
        const float q = u2f((uint32_t)b | 0x80000000u);
        int cp = 0, cq = 0;
        for (int k = 0; k < 15; ++k) {
            cp += p >= steps[k];
            cq += q >= steps[k];
        }
        bad += or_nf4_code_argmin(p) != cp;
        bad += or_nf4_code_argmin(q) != cq;
    }
    return bad;
}

/* quantizer.py:21-53. */
void or_quantize_nf4(const float *x, int64_t n, int32_t bs, uint8_t *packed,
                     float *absmax) {
    const int64_t nb = (n + bs - 1) / bs; /* zero padding, :30-34 */
    const int64_t npk = (n + 1) / 2;
    memset(packed, 0, (size_t)npk);
    for (int64_t b = 0; b < nb; ++b) {
        const int64_t s = b * bs;
        /* :35 absmax = max |x| over the padded block (pad zeros add 0). */
        float am = 0.0f;
        for (int64_t i = 0; i < bs; ++i) {
            float v = (s + i < n) ? fabsf(x[s + i]) : 0.0f;
            if (v > am || isnan(v)) am = v;
        }
        absmax[b] = am;                                 /* :48-53 unclamped */
        const float safe = (am < 1e-8f) ? 1e-8f : am;   /* :36 clamp(min=1e-8) */
        for (int64_t i = 0; i < bs && s + i < n; ++i) {
            const float nv = x[s + i] / safe;            /* :38 fp32 division */
            const uint8_t c = or_nf4_code_argmin(nv);    /* :40-41 */
            const int64_t e = s + i;                     /* :43-46 packing */
            if ((e & 1) == 0) packed[e >> 1] |= (uint8_t)(c << 4);
            else packed[e >> 1] |= c;
        }
    }
    /* :44-45 an odd count gets a code-0 pad nibble: already 0 from memset. */
}

/* Double-quant spec (the reference has none): scale = max/127 per group,
 * 1.0 when the group max is 0 (galore/src/quantize.rs:4-13); q =
 * clamp(rne(a / scale), 0, 127) with fp32 correctly rounded division. */
void or_dq_encode(const float *absmax, int64_t nblocks, int32_t group,
                  uint8_t *q, float *scale) {
    const int64_t ng = (nblocks + group - 1) / group;
    for (int64_t g = 0; g < ng; ++g) {
        const int64_t s = g * group;
        const int64_t e = (s + group < nblocks) ? s + group : nblocks;
        float mx = 0.0f;
        for (int64_t i = s; i < e; ++i) if (absmax[i] > mx) mx = absmax[i];
        const float sc = (mx <= 0.0f) ? 1.0f : mx / 127.0f;
        scale[g] = sc;
        for (int64_t i = s; i < e; ++i) {
            float r = rintf(absmax[i] / sc); /* default mode: half to even */
            if (!(r >= 0.0f)) r = 0.0f;
            if (r > 127.0f) r = 127.0f;
            q[i] = (uint8_t)r;
        }
    }
}

void or_dq_decode(const uint8_t *q, const float *scale, int64_t nblocks,
                  int32_t group, float *absmax_out) {
    for (int64_t i = 0; i < nblocks; ++i)
        absmax_out[i] = (float)q[i] * scale[i / group];
}

/* nf4.rs:37-83 core: returns 0 ok, 1 absmax too small, 2 packed too small. */
static int dequant_check(int64_t packed_len, int64_t absmax_len, int64_t n,
                         int32_t bs) {
    const int64_t nb = (n + bs - 1) / bs;                 /* :44 div_ceil */
    if (absmax_len < nb) return 1;                        /* :46-51 */
    if (packed_len * 2 < n) return 2;                     /* :52-57 */
    return 0;
}

static inline float nf4_value(const uint8_t *packed, int64_t e, float am) {
    const uint8_t byte = packed[e / 2];                    /* :66-69 */
    const uint8_t nib = (e % 2 == 0) ? (byte >> 4) & 0xf : byte & 0xf; /* :70-74 */
    return kCodes[nib] * am;                               /* :76-77 one fp32 mul */
}

int or_dequant_f32(const uint8_t *packed, int64_t packed_len,
                   const float *absmax, int64_t absmax_len, float *out,
                   int64_t n, int32_t bs) {
    int rc = dequant_check(packed_len, absmax_len, n, bs);
    if (rc) return rc;
    const int64_t nb = (n + bs - 1) / bs;
    for (int64_t b = 0; b < nb; ++b)                       /* :59-63 */
        for (int64_t e = b * bs; e < n && e < (b + 1) * bs; ++e)
            out[e] = nf4_value(packed, e, absmax[b]);
    return 0;
}

int or_dequant_f16(const uint8_t *packed, int64_t packed_len,
                   const float *absmax, int64_t absmax_len, uint16_t *out,
                   int64_t n, int32_t bs) {
    int rc = dequant_check(packed_len, absmax_len, n, bs);
    if (rc) return rc;
    const int64_t nb = (n + bs - 1) / bs;
    for (int64_t b = 0; b < nb; ++b)
        for (int64_t e = b * bs; e < n && e < (b + 1) * bs; ++e)
            out[e] = or_f32_to_f16(nf4_value(packed, e, absmax[b])); /* :78 */
    return 0;
}

int or_dequant_bf16(const uint8_t *packed, int64_t packed_len,
                    const float *absmax, int64_t absmax_len, uint16_t *out,
                    int64_t n, int32_t bs) {
    int rc = dequant_check(packed_len, absmax_len, n, bs);
    if (rc) return rc;
    const int64_t nb = (n + bs - 1) / bs;
    for (int64_t b = 0; b < nb; ++b)
        for (int64_t e = b * bs; e < n && e < (b + 1) * bs; ++e)
            out[e] = or_f32_to_bf16(nf4_value(packed, e, absmax[b]));
    return 0;
}

/* doublepass/src/math.rs:9-21. */
void or_matmul_tb(const float *a, const float *b, int64_t m, int64_t k,
                  int64_t n, float *c) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            float s = 0.0f;
            for (int64_t l = 0; l < k; ++l) s += a[i * k + l] * b[j * k + l];
            c[i * n + j] = s;
        }
}

/* doublepass/src/backward.rs:87-93 (d_wd[k*ff+j] += d_mlp_out[i*d+k] *
 * hidden[i*ff+j], outer loops over the gradient's element, inner over the
 * tokens i). */
void or_wgrad(const float *dy, const float *x, int64_t m, int64_t n,
              int64_t k, float *dw) {
    for (int64_t r = 0; r < n; ++r)
        for (int64_t c = 0; c < k; ++c)
            for (int64_t i = 0; i < m; ++i) dw[r * k + c] += dy[i * n + r] * x[i * k + c];
}

/* doublepass/src/backward.rs:160-168 (d_attn_out += d_out_proj . Wo); the
 * sites :79-85, :117-129 and :284-300 have the same shape. */
void or_dgrad(const float *dy, const float *w, int64_t m, int64_t n,
              int64_t k, float *dx) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            const float g = dy[i * n + j];
            for (int64_t l = 0; l < k; ++l) dx[i * k + l] += g * w[j * k + l];
        }
}

/* doublepass/src/math.rs:36-59: the sum of squares in index order, one fp32
 * division by d, sqrt(mean_sq + eps), then x / rms and * w per element. */
void or_rmsnorm_fwd(const float *x, const float *w, int64_t m, int64_t d, float eps,
                    float *y, float *x_hat, float *rms) {
    for (int64_t b = 0; b < m; ++b) {
        float s = 0.0f;
        for (int64_t i = 0; i < d; ++i) {
            const float v = x[b * d + i];
            const float sq = v * v;
            s += sq;
        }
        const float mean_sq = s / (float)d;
        const float r = sqrtf(mean_sq + eps);
        rms[b] = r;
        for (int64_t i = 0; i < d; ++i) {
            const float xh = x[b * d + i] / r;
            x_hat[b * d + i] = xh;
            y[b * d + i] = xh * w[i];
        }
    }
}

static inline uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

void or_gen_normal(uint64_t seed, int64_t n, double sigma, float *out) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        double u1 = 1.0 - (double)(splitmix64(&s) >> 11) * 0x1p-53; /* (0,1] */
        double u2 = (double)(splitmix64(&s) >> 11) * 0x1p-53;       /* [0,1) */
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(r * cos(two_pi * u2) * sigma);
        if (i + 1 < n) out[i + 1] = (float)(r * sin(two_pi * u2) * sigma);
    }
}
