/*
 * qmoe_oracle.c -- CPU restatement of the reference MoE FFN layer (test
 * infrastructure only; see qmoe_oracle.h for scope and citations).
 *
 * Build: oracle/Makefile (gcc -O3 -march=x86-64-v3 -ffp-contract=off -fopenmp).
 * -ffp-contract=off matters: every deterministic function below is a fixed
 * sequence of separately rounded IEEE operations.
 */
#include "qmoe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32 (ggml's GGML_FP32_TO_FP16 on F16C hardware is IEEE RNE)     */
/* ------------------------------------------------------------------------ */
uint16_t qo_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mant = x & 0x7fffffu;
    int exp = (int)((x >> 23) & 0xffu);
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? (0x200u | (mant >> 13)) : 0u));
    int e = exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t full = mant | 0x800000u;
        int shift = 14 - e;
        uint32_t half = full >> shift;
        uint32_t rem = full & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half & 1u))) half++;
        return (uint16_t)(sign | half);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

float qo_fp16_to_fp32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            m &= 0x3ffu;
            x = sign | ((uint32_t)(113 - sh) << 23) | (m << 13);
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

/* ------------------------------------------------------------------------ */
/* Deterministic elementary functions: fixed sequences of IEEE f64 ops.      */
/* ------------------------------------------------------------------------ */
static const double QO_LN2_HI = 6.93147180369123816490e-01; /* 32 significant bits */
static const double QO_LN2_LO = 1.90821492927058770002e-10;
static const double QO_LOG2E  = 1.44269504088896338700e+00;

double qo_exp_det(double x) {
    if (x != x) return x;
    if (x > 709.78) return INFINITY;
    if (x < -745.2) return 0.0;
    double k = rint(x * QO_LOG2E);
    double r = x - k * QO_LN2_HI;
    r = r - k * QO_LN2_LO;
    /* Taylor series of exp(r), |r| <= 0.347, degree 13 (error < 1e-17) */
    double p = 1.0 / 6227020800.0;
    p = p * r + 1.0 / 479001600.0;
    p = p * r + 1.0 / 39916800.0;
    p = p * r + 1.0 / 3628800.0;
    p = p * r + 1.0 / 362880.0;
    p = p * r + 1.0 / 40320.0;
    p = p * r + 1.0 / 5040.0;
    p = p * r + 1.0 / 720.0;
    p = p * r + 1.0 / 120.0;
    p = p * r + 1.0 / 24.0;
    p = p * r + 1.0 / 6.0;
    p = p * r + 0.5;
    p = p * r + 1.0;
    p = p * r + 1.0;
    return ldexp(p, (int)k);
}

double qo_log_det(double x) {
    int e;
    double m = frexp(x, &e); /* x = m * 2^e, m in [0.5, 1) */
    if (m < 0.70710678118654752440) { m = m * 2.0; e = e - 1; }
    double s = (m - 1.0) / (m + 1.0);
    double s2 = s * s;
    double p = 1.0 / 23.0;
    p = p * s2 + 1.0 / 21.0;
    p = p * s2 + 1.0 / 19.0;
    p = p * s2 + 1.0 / 17.0;
    p = p * s2 + 1.0 / 15.0;
    p = p * s2 + 1.0 / 13.0;
    p = p * s2 + 1.0 / 11.0;
    p = p * s2 + 1.0 / 9.0;
    p = p * s2 + 1.0 / 7.0;
    p = p * s2 + 1.0 / 5.0;
    p = p * s2 + 1.0 / 3.0;
    p = p * s2 + 1.0;
    double de = (double)e;
    return de * QO_LN2_HI + (de * QO_LN2_LO + 2.0 * s * p);
}

double qo_cospi2_det(double u) {
    double t = u * 4.0;
    double q = floor(t);
    double f = t - q;
    if (f > 0.5) { f = f - 1.0; q = q + 1.0; }
    double a = f * 1.57079632679489661923; /* |a| <= pi/4 */
    double a2 = a * a;
    double c = 1.0 / 20922789888000.0;      /* 1/16! */
    c = c * a2 - 1.0 / 87178291200.0;       /* 1/14! */
    c = c * a2 + 1.0 / 479001600.0;         /* 1/12! */
    c = c * a2 - 1.0 / 3628800.0;           /* 1/10! */
    c = c * a2 + 1.0 / 40320.0;
    c = c * a2 - 1.0 / 720.0;
    c = c * a2 + 1.0 / 24.0;
    c = c * a2 - 0.5;
    c = c * a2 + 1.0;
    double s = 1.0 / 355687428096000.0;     /* 1/17! */
    s = s * a2 - 1.0 / 1307674368000.0;     /* 1/15! */
    s = s * a2 + 1.0 / 6227020800.0;        /* 1/13! */
    s = s * a2 - 1.0 / 39916800.0;          /* 1/11! */
    s = s * a2 + 1.0 / 362880.0;
    s = s * a2 - 1.0 / 5040.0;
    s = s * a2 + 1.0 / 120.0;
    s = s * a2 - 1.0 / 6.0;
    s = s * a2 + 1.0;
    s = s * a;
    switch (((int)q) & 3) {
        case 0: return c;
        case 1: return -s;
        case 2: return -c;
        default: return s;
    }
}

/* ------------------------------------------------------------------------ */
/* Counter-based RNG: splitmix64 finalizer over (seed, stream, counter).     */
/* ------------------------------------------------------------------------ */
static uint64_t qo_mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t qo_hash3(uint64_t seed, uint64_t stream, uint64_t ctr) {
    uint64_t key = qo_mix64(seed ^ qo_mix64(stream + 0x632BE59BD9B4E019ull));
    return qo_mix64(key ^ ctr);
}

double qo_normal(uint64_t seed, uint64_t stream, uint64_t idx) {
    uint64_t h1 = qo_hash3(seed, stream, 2 * idx);
    uint64_t h2 = qo_hash3(seed, stream, 2 * idx + 1);
    double u1 = (double)((h1 >> 11) + 1) * (1.0 / 9007199254740992.0); /* (0,1] */
    double u2 = (double)(h2 >> 11) * (1.0 / 9007199254740992.0);       /* [0,1) */
    double r = sqrt(-2.0 * qo_log_det(u1));
    return r * qo_cospi2_det(u2);
}

void qo_gen_normal_f32(uint64_t seed, uint64_t stream, double mean, double sigma,
                       float* out, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        out[i] = (float)(mean + sigma * qo_normal(seed, stream, (uint64_t)i));
    }
}

/* ------------------------------------------------------------------------ */
/* Block formats                                                             */
/* ------------------------------------------------------------------------ */
size_t qo_type_block_bytes(int type) {
    switch (type) {
        case QO_TYPE_Q4_0: return 18;
        case QO_TYPE_Q8_0: return 34;
        case QO_TYPE_F32: return 4;
        default: return 0;
    }
}

size_t qo_row_bytes(int type, int64_t n) {
    if (type == QO_TYPE_F32) return (size_t)n * 4;
    return (size_t)(n / 32) * qo_type_block_bytes(type);
}

static void put_u16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)(v & 0xff); p[1] = (uint8_t)(v >> 8); }
static uint16_t get_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

void qo_quantize_q4_0(const float* x, void* dst, int64_t n) {
    uint8_t* out = (uint8_t*)dst;
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* xb = x + b * 32;
        uint8_t* yb = out + b * 18;
        float amax = 0.0f, vmax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            float v = xb[j];
            if (amax < fabsf(v)) { amax = fabsf(v); vmax = v; }
        }
        const float d = vmax / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        put_u16(yb, qo_fp32_to_fp16(d));
        for (int j = 0; j < 16; ++j) {
            const float x0 = xb[j] * id;
            const float x1 = xb[16 + j] * id;
            int xi0 = (int)(int8_t)(int)(x0 + 8.5f);
            int xi1 = (int)(int8_t)(int)(x1 + 8.5f);
            if (xi0 > 15) xi0 = 15;
            if (xi1 > 15) xi1 = 15;
            yb[2 + j] = (uint8_t)(xi0 | (xi1 << 4));
        }
    }
}

void qo_quantize_q8_0(const float* x, void* dst, int64_t n) {
    uint8_t* out = (uint8_t*)dst;
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* xb = x + b * 32;
        uint8_t* yb = out + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            float v = fabsf(xb[j]);
            if (v > amax) amax = v;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        put_u16(yb, qo_fp32_to_fp16(d));
        for (int j = 0; j < 32; ++j) {
            yb[2 + j] = (uint8_t)(int8_t)roundf(xb[j] * id);
        }
    }
}

void qo_quantize_q8_0_act(const float* x, void* dst, int64_t n) {
    uint8_t* out = (uint8_t*)dst;
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* xb = x + b * 32;
        uint8_t* yb = out + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            float v = fabsf(xb[j]);
            if (v > amax) amax = v;
        }
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        put_u16(yb, qo_fp32_to_fp16(d));
        for (int j = 0; j < 32; ++j) {
            yb[2 + j] = (uint8_t)(int8_t)(int)nearbyintf(xb[j] * id);
        }
    }
}

void qo_dequantize(int type, const void* src, float* dst, int64_t n) {
    const uint8_t* in = (const uint8_t*)src;
    if (type == QO_TYPE_F32) { memcpy(dst, src, (size_t)n * 4); return; }
    for (int64_t b = 0; b < n / 32; ++b) {
        if (type == QO_TYPE_Q4_0) {
            const uint8_t* blk = in + b * 18;
            const float d = qo_fp16_to_fp32(get_u16(blk));
            for (int j = 0; j < 16; ++j) {
                dst[b * 32 + j] = (float)((int)(blk[2 + j] & 0x0f) - 8) * d;
                dst[b * 32 + 16 + j] = (float)((int)(blk[2 + j] >> 4) - 8) * d;
            }
        } else {
            const uint8_t* blk = in + b * 34;
            const float d = qo_fp16_to_fp32(get_u16(blk));
            for (int j = 0; j < 32; ++j) dst[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
        }
    }
}

double qo_vec_dot_f64(int wtype, const void* wrow, const void* xq8, int64_t n) {
    const uint8_t* w = (const uint8_t*)wrow;
    const uint8_t* xq = (const uint8_t*)xq8;
    double acc = 0.0;
    for (int64_t b = 0; b < n / 32; ++b) {
        const uint8_t* xb = xq + b * 34;
        const int8_t* xs = (const int8_t*)(xb + 2);
        const float dx = qo_fp16_to_fp32(get_u16(xb));
        int32_t isum = 0;
        float dw;
        if (wtype == QO_TYPE_Q4_0) {
            const uint8_t* wb = w + b * 18;
            dw = qo_fp16_to_fp32(get_u16(wb));
            for (int j = 0; j < 16; ++j) {
                isum += ((int)(wb[2 + j] & 0x0f) - 8) * (int)xs[j];
                isum += ((int)(wb[2 + j] >> 4) - 8) * (int)xs[16 + j];
            }
        } else {
            const uint8_t* wb = w + b * 34;
            const int8_t* ws = (const int8_t*)(wb + 2);
            dw = qo_fp16_to_fp32(get_u16(wb));
            for (int j = 0; j < 32; ++j) isum += (int)ws[j] * (int)xs[j];
        }
        /* fp32(d_w)*fp32(d_x) is exact in f32 (two 11-bit significands) */
        const float dd = dw * dx;
        acc += (double)dd * (double)isum;
    }
    return acc;
}

float qo_vec_dot(int wtype, const void* wrow, const void* xq8, int64_t n) {
    return (float)qo_vec_dot_f64(wtype, wrow, xq8, n);
}

/* ------------------------------------------------------------------------ */
/* Router, top-k, softmax, assignment sort                                   */
/* ------------------------------------------------------------------------ */
float qo_dot_f32_exact(const float* a, const float* b, int64_t n) {
    double acc = 0.0;
    for (int64_t i = 0; i < n; ++i) acc += (double)a[i] * (double)b[i];
    return (float)acc;
}

void qo_router_logits(const float* w_router, const float* x, int T, int H, int E, float* logits) {
#pragma omp parallel for schedule(static)
    for (int64_t te = 0; te < (int64_t)T * E; ++te) {
        const int t = (int)(te / E), e = (int)(te % E);
        logits[te] = qo_dot_f32_exact(w_router + (size_t)e * H, x + (size_t)t * H, H);
    }
}

void qo_topk_softmax(const float* logits, int T, int E, int k, int32_t* idx, float* w) {
    for (int t = 0; t < T; ++t) {
        const float* l = logits + (size_t)t * E;
        int32_t* it = idx + (size_t)t * k;
        /* selection with ties to the lowest index (argsort DESC, stable) */
        for (int j = 0; j < k; ++j) {
            int best = -1;
            for (int e = 0; e < E; ++e) {
                int taken = 0;
                for (int jj = 0; jj < j; ++jj) if (it[jj] == e) { taken = 1; break; }
                if (taken) continue;
                if (best < 0 || l[e] > l[best]) best = e;
            }
            it[j] = best;
        }
        /* softmax over the selected logits (moe.cpp:88-94); max is slot 0 */
        double ex[64];
        double m = (double)l[it[0]], sum = 0.0;
        for (int j = 0; j < k; ++j) { ex[j] = qo_exp_det((double)l[it[j]] - m); sum += ex[j]; }
        for (int j = 0; j < k; ++j) w[(size_t)t * k + j] = (float)(ex[j] / sum);
    }
}

void qo_sort_assignments(const int32_t* idx, int T, int E, int k,
                         int32_t* offsets, int32_t* rows, int32_t* pos) {
    int32_t* fill = (int32_t*)calloc((size_t)E + 1, sizeof(int32_t));
    for (int e = 0; e <= E; ++e) offsets[e] = 0;
    for (int64_t a = 0; a < (int64_t)T * k; ++a) offsets[idx[a] + 1]++;
    for (int e = 0; e < E; ++e) offsets[e + 1] += offsets[e];
    for (int t = 0; t < T; ++t) {
        for (int j = 0; j < k; ++j) {
            const int64_t a = (int64_t)t * k + j;
            const int e = idx[a];
            const int32_t p = offsets[e] + fill[e]++;
            rows[p] = (int32_t)a;
            if (pos) pos[a] = p;
        }
    }
    free(fill);
}

float qo_silu_mul(float g, float u) {
    const double gd = (double)g;
    const double s = gd / (1.0 + qo_exp_det(-gd));
    return (float)(s * (double)u);
}

/* gelu_f32 of ggml (the value its CPU table stores before the fp16 rounding);
 * the C expression parses as ((0.5f*x) * (1 + tanhf(((c*x) * (1 + ((a*x)*x)))))). */
static float qo_gelu_tanh_f32(float x) {
    const float a = 0.044715f;
    const float c = 0.79788456080286535587989211986876f; /* sqrt(2/pi) */
    return 0.5f * x * (1.0f + tanhf(c * x * (1.0f + a * x * x)));
}

float qo_gelu_f16(float x) {
    if (x <= -10.0f) return 0.0f;
    if (x >= 10.0f) return x;
    const float xh = qo_fp16_to_fp32(qo_fp32_to_fp16(x));
    return qo_fp16_to_fp32(qo_fp32_to_fp16(qo_gelu_tanh_f32(xh)));
}

float qo_geglu_mul(float g, float u) { return qo_gelu_f16(g) * u; }

static float qo_act_mul(int act, float g, float u) {
    return act == QO_ACT_GELU_TANH ? qo_geglu_mul(g, u) : qo_silu_mul(g, u);
}

float qo_sigmoid(float g) {
    return (float)(1.0 / (1.0 + qo_exp_det(-(double)g)));
}

void qo_rms_norm(const float* x, const float* w, int T, int H, float eps, float* y) {
    for (int t = 0; t < T; ++t) {
        const float* xt = x + (size_t)t * H;
        double sum = 0.0;
        for (int i = 0; i < H; ++i) sum += (double)(xt[i] * xt[i]);
        const float mean = (float)(sum / (double)H);
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int i = 0; i < H; ++i) {
            const float v = xt[i] * scale;
            y[(size_t)t * H + i] = w ? v * w[i] : v;
        }
    }
}

void qo_rms_partials(const float* x, int T, int H, double* out) {
    const int np = (H + 31) / 32;
    for (int t = 0; t < T; ++t) {
        const float* xt = x + (size_t)t * H;
        for (int c = 0; c < np; ++c) {
            double r[8];
            for (int j = 0; j < 8; ++j) {
                double s = 0.0;
                for (int k = 0; k < 4; ++k) {
                    const int col = 32 * c + 4 * j + k;
                    if (col < H) {
                        const float q = xt[col] * xt[col];
                        s += (double)q;
                    }
                }
                r[j] = s;
            }
            out[(size_t)t * np + c] = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        }
    }
}

void qo_gemma4_moe_inputs(const float* x, const float* w_pre, const float* w_rs, int T, int H, float eps,
                          float* expert_in, float* router_in) {
    const float s = 1.0f / sqrtf((float)H);
    for (int t = 0; t < T; ++t) {
        const float* xt = x + (size_t)t * H;
        double sum = 0.0;
        for (int i = 0; i < H; ++i) sum += (double)(xt[i] * xt[i]);
        const float mean = (float)(sum / (double)H);
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int i = 0; i < H; ++i) {
            const float v = xt[i] * scale;
            expert_in[(size_t)t * H + i] = v * w_pre[i];
            const float r = v * s;
            router_in[(size_t)t * H + i] = r * w_rs[i];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Whole layer: router -> top-k -> expert-major grouped SwiGLU -> combine    */
/* ------------------------------------------------------------------------ */
int qo_moe_forward(const qo_layer* L, const float* x, int T, float* y,
                   qo_debug* dbg, int nthreads) {
    return qo_moe_forward_routed(L, x, x, T, y, dbg, nthreads);
}

int qo_moe_forward_routed(const qo_layer* L, const float* x, const float* xr, int T, float* y,
                          qo_debug* dbg, int nthreads) {
    if (!L || !x || !xr || !y || T < 0) return 1;
    const int H = L->n_embd, E = L->n_experts, k = L->top_k, F = L->ffn_dim;
    const int wt = L->expert_type;
    if (H % 32 || F % 32 || k < 1 || k > E || k > 64) return 2;
    if (wt != QO_TYPE_Q4_0 && wt != QO_TYPE_Q8_0) return 3;
    if (T == 0) return 0;
#ifdef _OPENMP
    int saved_threads = omp_get_max_threads();
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    const size_t xq_row = qo_row_bytes(QO_TYPE_Q8_0, H);
    const size_t hq_row = qo_row_bytes(QO_TYPE_Q8_0, F);
    const size_t wrow_h = qo_row_bytes(wt, H);   /* gate/up row */
    const size_t wrow_f = qo_row_bytes(wt, F);   /* down row */
    const int64_t A = (int64_t)T * k;

    float* logits = (float*)malloc(sizeof(float) * (size_t)T * E);
    int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * (size_t)A);
    float* wts = (float*)malloc(sizeof(float) * (size_t)A);
    int32_t* offsets = (int32_t*)malloc(sizeof(int32_t) * ((size_t)E + 1));
    int32_t* rows = (int32_t*)malloc(sizeof(int32_t) * (size_t)A);
    uint8_t* xq = (uint8_t*)malloc(xq_row * (size_t)T);
    float* h = (float*)malloc(sizeof(float) * (size_t)A * F);
    uint8_t* hq = (uint8_t*)malloc(hq_row * (size_t)A);
    float* yd = (float*)malloc(sizeof(float) * (size_t)A * H);

    /* 1. router logits (moe.cpp:72), top-k (:77-82), softmax (:88-94) */
    qo_router_logits(L->w_router, xr, T, H, E, logits);
    qo_topk_softmax(logits, T, E, k, idx, wts);
    qo_sort_assignments(idx, T, E, k, offsets, rows, NULL);

    /* activation quantization (done inside ggml mul_mat_id for src1) */
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) qo_quantize_q8_0_act(x + (size_t)t * H, xq + xq_row * t, H);

    /* 2. gate/up mul_mat_id (moe.cpp:105-113) + silu*up (:117) or gelu*up
     *    (gemma4.cpp:419-423), expert-major */
    const int act = L->act;
    const size_t gu_rows = L->gate_up_fused ? 2 * (size_t)F : (size_t)F;  /* rows per expert */
    const uint8_t* w_up_base = L->gate_up_fused ? (const uint8_t*)L->w_gate + (size_t)F * wrow_h
                                                : (const uint8_t*)L->w_up;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t ef = 0; ef < (int64_t)E * (F / 32); ++ef) {
        const int e = (int)(ef / (F / 32));
        const int f0 = (int)(ef % (F / 32)) * 32;
        for (int p = offsets[e]; p < offsets[e + 1]; ++p) {
            const int64_t a = rows[p];
            const int t = (int)(a / k);
            for (int f = f0; f < f0 + 32; ++f) {
                const uint8_t* wg = (const uint8_t*)L->w_gate + ((size_t)e * gu_rows + f) * wrow_h;
                const uint8_t* wu = w_up_base + ((size_t)e * gu_rows + f) * wrow_h;
                const float g = qo_vec_dot(wt, wg, xq + xq_row * t, H);
                const float u = qo_vec_dot(wt, wu, xq + xq_row * t, H);
                h[a * F + f] = qo_act_mul(act, g, u);
            }
        }
    }
#pragma omp parallel for schedule(static)
    for (int64_t a = 0; a < A; ++a) qo_quantize_q8_0_act(h + a * F, hq + hq_row * a, F);

    /* 3. down mul_mat_id (moe.cpp:127), expert-major */
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t en = 0; en < (int64_t)E * (H / 32); ++en) {
        const int e = (int)(en / (H / 32));
        const int n0 = (int)(en % (H / 32)) * 32;
        for (int p = offsets[e]; p < offsets[e + 1]; ++p) {
            const int64_t a = rows[p];
            for (int n = n0; n < n0 + 32; ++n) {
                const uint8_t* wd = (const uint8_t*)L->w_down + ((size_t)e * H + n) * wrow_f;
                yd[a * H + n] = qo_vec_dot(wt, wd, hq + hq_row * a, F);
            }
        }
    }

    /* 4. weighted k-ordered sum (moe.cpp:134-151), then shared expert (:161-174) */
    float* sh_out = NULL;
    float* sh_gate = NULL;
    if (L->has_shared_expert) {
        sh_out = (float*)malloc(sizeof(float) * (size_t)T * H);
        sh_gate = (float*)malloc(sizeof(float) * (size_t)T);
#pragma omp parallel for schedule(static)
        for (int t = 0; t < T; ++t) {
            float* hs = (float*)malloc(sizeof(float) * (size_t)F);
            uint8_t* hsq = (uint8_t*)malloc(hq_row);
            for (int f = 0; f < F; ++f) {
                const float g = qo_vec_dot(wt, (const uint8_t*)L->w_sh_gate + (size_t)f * wrow_h, xq + xq_row * t, H);
                const float u = qo_vec_dot(wt, (const uint8_t*)L->w_sh_up + (size_t)f * wrow_h, xq + xq_row * t, H);
                hs[f] = qo_act_mul(act, g, u);
            }
            if (dbg && dbg->sh_h) memcpy(dbg->sh_h + (size_t)t * F, hs, sizeof(float) * (size_t)F);
            qo_quantize_q8_0_act(hs, hsq, F);
            for (int n = 0; n < H; ++n)
                sh_out[(size_t)t * H + n] = qo_vec_dot(wt, (const uint8_t*)L->w_sh_down + (size_t)n * wrow_f, hsq, F);
            sh_gate[t] = qo_sigmoid(qo_dot_f32_exact(L->w_sh_norm, xr + (size_t)t * H, H));
            free(hs);
            free(hsq);
        }
    }
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
        for (int n = 0; n < H; ++n) {
            float acc = wts[(size_t)t * k] * yd[((int64_t)t * k) * H + n];
            for (int j = 1; j < k; ++j) {
                const float term = wts[(size_t)t * k + j] * yd[((int64_t)t * k + j) * H + n];
                acc = acc + term;
            }
            if (L->has_shared_expert) {
                const float sc = sh_out[(size_t)t * H + n] * sh_gate[t];
                acc = acc + sc;
            }
            y[(size_t)t * H + n] = acc;
        }
    }

    if (dbg) {
        if (dbg->logits) memcpy(dbg->logits, logits, sizeof(float) * (size_t)T * E);
        if (dbg->topk_idx) memcpy(dbg->topk_idx, idx, sizeof(int32_t) * (size_t)A);
        if (dbg->topk_w) memcpy(dbg->topk_w, wts, sizeof(float) * (size_t)A);
        if (dbg->offsets) memcpy(dbg->offsets, offsets, sizeof(int32_t) * ((size_t)E + 1));
        if (dbg->rows) memcpy(dbg->rows, rows, sizeof(int32_t) * (size_t)A);
        if (dbg->h) memcpy(dbg->h, h, sizeof(float) * (size_t)A * F);
        if (dbg->y) memcpy(dbg->y, yd, sizeof(float) * (size_t)A * H);
        if (dbg->sh_gate && sh_gate) memcpy(dbg->sh_gate, sh_gate, sizeof(float) * (size_t)T);
        if (dbg->sh_out && sh_out) memcpy(dbg->sh_out, sh_out, sizeof(float) * (size_t)T * H);
    }
    free(logits); free(idx); free(wts); free(offsets); free(rows);
    free(xq); free(h); free(hq); free(yd); free(sh_out); free(sh_gate);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(saved_threads);
#endif
    return 0;
}
