/*
 * ubridge_oracle.c -- CPU restatement of Ubridge's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  See the header
 * for which test pins each function.  Compiled with -ffp-contract=off so that
 * every multiply and add rounds on its own, as the reference's separate
 * vmul / vsub vector ops do.
 */
#include "ubridge_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* scalar conversions                                                   */
/* ------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        /* subnormal: m * 2^-24, exact in f32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000 | (m << 13));
    return u2f(sign | ((e + 112) << 23) | (m << 13));
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000;
    uint32_t ax = x & 0x7fffffff;
    if (ax >= 0x7f800000) return (uint16_t)(sign | (ax > 0x7f800000 ? 0x7e00 : 0x7c00));
    if (ax < 0x38800000) { /* below 2^-14: f16 subnormal, step 2^-24 */
        if (ax < 0x33000000) return (uint16_t)sign; /* < 2^-25 */
        uint32_t e = ax >> 23, m = (ax & 0x7fffff) | 0x800000;
        uint32_t shift = 126 - e;
        uint32_t r = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (ax - 0x38000000) >> 13, rem = ax & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (r & 1))) r++;
    if (r >= 0x7c00) r = 0x7c00;
    return (uint16_t)(sign | r);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t orc_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7fffffff) > 0x7f800000) return (uint16_t)((x >> 16) | 0x40);
    x += 0x7fff + ((x >> 16) & 1);
    return (uint16_t)(x >> 16);
}

void orc_f32_to_bf16_n(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(in[i]);
}
void orc_bf16_to_f32_n(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_bf16_to_f32(in[i]);
}

/* OCP FP8 e4m3fn: bias 7, no infinities, 0x7f/0xff NaN, max 448. */
float orc_e4m3_to_f32(uint8_t v) {
    int sign = v & 0x80, e = (v >> 3) & 0xf, m = v & 7;
    float r;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) r = (float)m * 0.001953125f; /* m * 2^-9 */
    else r = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return sign ? -r : r;
}

uint8_t orc_f32_to_e4m3(float f) {
    uint8_t sign = (f2u(f) >> 24) & 0x80;
    if (isnan(f)) return sign | 0x7f;
    float a = fabsf(f);
    if (a >= 448.0f) return sign | 0x7e;
    if (a < 0.015625f) { /* subnormal range, step 2^-9; 8 * 2^-9 encodes min normal 0x08 */
        float q = nearbyintf(a * 512.0f);
        return sign | (uint8_t)q;
    }
    int e2;
    float fr = frexpf(a, &e2); /* a = fr * 2^e2, fr in [0.5,1) */
    int e = e2 - 1;
    float mant = fr * 2.0f; /* [1,2) */
    int q = (int)nearbyintf((mant - 1.0f) * 8.0f);
    if (q == 8) { q = 0; e++; }
    int code = ((e + 7) << 3) | q;
    if (code > 0x7e) code = 0x7e;
    return sign | (uint8_t)code;
}

static inline float to_float_dt(const void* p, size_t i, int dt) {
    if (dt == ORC_F32) return ((const float*)p)[i];
    if (dt == ORC_F16) return orc_f16_to_f32(((const uint16_t*)p)[i]);
    return orc_bf16_to_f32(((const uint16_t*)p)[i]);
}
static inline void store_dt(void* p, size_t i, float v, int dt) {
    if (dt == ORC_F32) ((float*)p)[i] = v;
    else if (dt == ORC_F16) ((uint16_t*)p)[i] = orc_f32_to_f16(v);
    else ((uint16_t*)p)[i] = orc_f32_to_bf16(v);
}

/* ------------------------------------------------------------------ */
/* GGUF dequant, SoA layout                                             */
/* ------------------------------------------------------------------ */

/* Q8_0: SoA "[nb x fp16 d][nb x 32 int8]" (quant.cpp:217-220).
 * Per element the reference converts the fp16 scale to T first
 * (quant.cpp:250 convert<T,__fp16>), casts q to T and multiplies in T
 * (quant.cpp:199-208).  f32 and f16: one rounding of the exact product.
 * bf16: bf16(bf16(d) * q) -- the scale is rounded to bf16 before the mul. */
void orc_dequant_q8_0(const uint8_t* in, void* out, size_t numel, int dt) {
    size_t nb = (numel + 31) / 32;
    const uint16_t* d = (const uint16_t*)in;
    const int8_t* q = (const int8_t*)(in + nb * 2);
    for (size_t i = 0; i < numel; i++) {
        float df = orc_f16_to_f32(d[i / 32]);
        if (dt == ORC_BF16) df = orc_bf16_to_f32(orc_f32_to_bf16(df));
        store_dt(out, i, df * (float)q[i], dt);
    }
}

/* Q4_0 (block_q4_0, quant.cpp:64-70; the reference ships no Q4_0 kernel):
 * SoA "[nb x fp16 d][nb x 16 B qs]", GGML nibble order: byte j low nibble is
 * element j, high nibble element j+16; x = (q - 8) * d, rounded once to T. */
void orc_dequant_q4_0(const uint8_t* in, void* out, size_t numel, int dt) {
    size_t nb = numel / 32;
    const uint16_t* d = (const uint16_t*)in;
    const uint8_t* qs = in + nb * 2;
    for (size_t b = 0; b < nb; b++) {
        float df = orc_f16_to_f32(d[b]);
        for (int j = 0; j < 16; j++) {
            uint8_t byte = qs[b * 16 + j];
            store_dt(out, b * 32 + j, (float)((int)(byte & 0xF) - 8) * df, dt);
            store_dt(out, b * 32 + j + 16, (float)((int)(byte >> 4) - 8) * df, dt);
        }
    }
}

/* get_scale_min_k4 (quant.cpp:356-363). */
static inline void scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
    }
}

/* Q4_K: SoA "[nb x 16 B header {fp16 d, fp16 dmin, u8 scales[12]}][nb x 128 B qs]"
 * (quant.cpp:366-370,439-442).  Values follow GGML dequantize_row_q4_K: for
 * each 64-element group j, scales/mins (is, is+1); y = d*sc*q_lo - dmin*m for
 * the low nibbles of 32 bytes, d*sc2*q_hi - dmin*m2 for the high nibbles.
 * The reference kernel (quant.cpp:372-430) deviates from this -- it applies
 * m1 to both halves (:412), reads 64 of the 128 qs bytes (:389) and stores v1
 * twice (:419-420) -- those are bugs, not the format, and are not restated. */
void orc_dequant_q4_k(const uint8_t* in, void* out, size_t numel, int dt) {
    size_t nb = numel / 256;
    const uint8_t* hdr = in;
    const uint8_t* qsall = in + nb * 16;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* h = hdr + b * 16;
        uint16_t dh, mh;
        memcpy(&dh, h, 2);
        memcpy(&mh, h + 2, 2);
        float d = orc_f16_to_f32(dh), dmin = orc_f16_to_f32(mh);
        const uint8_t* sc = h + 4;
        const uint8_t* q = qsall + b * 128;
        size_t o = b * 256;
        for (int j = 0, is = 0; j < 256; j += 64, is += 2) {
            uint8_t s, m;
            scale_min_k4(is, sc, &s, &m);
            float d1 = d * (float)s, m1 = dmin * (float)m;
            scale_min_k4(is + 1, sc, &s, &m);
            float d2 = d * (float)s, m2 = dmin * (float)m;
            for (int l = 0; l < 32; l++) store_dt(out, o + l, d1 * (float)(q[l] & 0xF) - m1, dt);
            for (int l = 0; l < 32; l++) store_dt(out, o + 32 + l, d2 * (float)(q[l] >> 4) - m2, dt);
            q += 32;
            o += 64;
        }
    }
}

/* GGUF AoS block sizes: q4_0 18 B {d, qs[16]}, q8_0 34 B {d, qs[32]},
 * q4_K 144 B {d, dmin, scales[12], qs[128]} (quant.cpp:64-70,98-104,144-151). */
static void soa_geom(int qt, size_t* head, size_t* body) {
    if (qt == ORC_Q4_0) { *head = 2; *body = 16; }
    else if (qt == ORC_Q8_0) { *head = 2; *body = 32; }
    else { *head = 16; *body = 128; }
}
void orc_aos_to_soa(int qt, const uint8_t* aos, uint8_t* soa, size_t nb) {
    size_t h, b;
    soa_geom(qt, &h, &b);
    for (size_t i = 0; i < nb; i++) {
        memcpy(soa + i * h, aos + i * (h + b), h);
        memcpy(soa + nb * h + i * b, aos + i * (h + b) + h, b);
    }
}
void orc_soa_to_aos(int qt, const uint8_t* soa, uint8_t* aos, size_t nb) {
    size_t h, b;
    soa_geom(qt, &h, &b);
    for (size_t i = 0; i < nb; i++) {
        memcpy(aos + i * (h + b), soa + i * h, h);
        memcpy(aos + i * (h + b) + h, soa + nb * h + i * b, b);
    }
}

/* ------------------------------------------------------------------ */
/* activation quantization (Candle k_quants BlockQ8_0/BlockQ8K from_float) */
/* ------------------------------------------------------------------ */

/* Q8_0: d = amax/127, id = 1/d, q = round-half-away(x*id), d stored fp16.
 * The reference's quantize_q8_0 (quant.cpp:270-290) takes amax over the first
 * 16 lanes of each 32-block only (:279-280, a 16-lane load of a 32-block); the
 * full-block amax of GGML/Candle is restated instead. */
void orc_quantize_q8_0(const float* x, size_t n, uint8_t* soa) {
    size_t nb = n / 32;
    uint16_t* dout = (uint16_t*)soa;
    int8_t* qout = (int8_t*)(soa + nb * 2);
    for (size_t b = 0; b < nb; b++) {
        const float* xb = x + b * 32;
        float amax = 0.f;
        for (int j = 0; j < 32; j++) {
            float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        float d = amax / 127.0f;
        float id = d != 0.f ? 1.0f / d : 0.f;
        dout[b] = orc_f32_to_f16(d);
        for (int j = 0; j < 32; j++) qout[b * 32 + j] = (int8_t)roundf(xb[j] * id);
    }
}

/* Q8_K: max = signed value of largest |x| (first wins), iscale = -128/max,
 * q = min(127, round(iscale*x)), bsums over 16, d = 1/iscale. */
void orc_quantize_q8_k(const float* x, size_t n, float* d, int8_t* qs, int16_t* bsums) {
    size_t nb = n / 256;
    for (size_t b = 0; b < nb; b++) {
        const float* xb = x + b * 256;
        float max = 0.f, amax = 0.f;
        for (int j = 0; j < 256; j++) {
            float a = fabsf(xb[j]);
            if (amax < a) { amax = a; max = xb[j]; }
        }
        if (amax == 0.f) {
            d[b] = 0.f;
            memset(qs + b * 256, 0, 256);
            memset(bsums + b * 16, 0, 32);
            continue;
        }
        float iscale = -128.0f / max;
        for (int j = 0; j < 256; j++) {
            float v = roundf(iscale * xb[j]);
            if (v > 127.f) v = 127.f;
            qs[b * 256 + j] = (int8_t)v;
        }
        for (int j = 0; j < 16; j++) {
            int s = 0;
            for (int i = 0; i < 16; i++) s += qs[b * 256 + j * 16 + i];
            bsums[b * 16 + j] = (int16_t)s;
        }
        d[b] = 1.0f / iscale;
    }
}

/* ------------------------------------------------------------------ */
/* Candle CPU QMatMul (k_quants::matmul + generic vec_dot)              */
/* ------------------------------------------------------------------ */

/* vec_dot Q4_0 x Q8_0: sumf += (float)sumi * d_w * d_a per block. */
static float vec_dot_q4_0(int K, const uint8_t* w, size_t wb0, size_t nbw, const uint8_t* a,
                          size_t nba) {
    const uint16_t* wd = (const uint16_t*)w;
    const uint8_t* wq = w + nbw * 2;
    const uint16_t* ad = (const uint16_t*)a;
    const int8_t* aq = (const int8_t*)(a + nba * 2);
    float sumf = 0.f;
    for (int b = 0; b < K / 32; b++) {
        const uint8_t* q = wq + (wb0 + b) * 16;
        const int8_t* y = aq + (size_t)b * 32;
        int sumi = 0;
        for (int j = 0; j < 16; j++) {
            int v0 = (q[j] & 0xF) - 8, v1 = (q[j] >> 4) - 8;
            sumi += v0 * y[j] + v1 * y[j + 16];
        }
        sumf += (float)sumi * orc_f16_to_f32(wd[wb0 + b]) * orc_f16_to_f32(ad[b]);
    }
    return sumf;
}

static float vec_dot_q8_0(int K, const uint8_t* w, size_t wb0, size_t nbw, const uint8_t* a,
                          size_t nba) {
    const uint16_t* wd = (const uint16_t*)w;
    const int8_t* wq = (const int8_t*)(w + nbw * 2);
    const uint16_t* ad = (const uint16_t*)a;
    const int8_t* aq = (const int8_t*)(a + nba * 2);
    float sumf = 0.f;
    for (int b = 0; b < K / 32; b++) {
        const int8_t* q = wq + (wb0 + b) * 32;
        const int8_t* y = aq + (size_t)b * 32;
        int sumi = 0;
        for (int j = 0; j < 32; j++) sumi += q[j] * y[j];
        sumf += (float)sumi * orc_f16_to_f32(wd[wb0 + b]) * orc_f16_to_f32(ad[b]);
    }
    return sumf;
}

/* vec_dot Q4_K x Q8_K, the generic (non-SIMD) form of GGML / Candle. */
static float vec_dot_q4_k(int K, const uint8_t* w, size_t wb0, size_t nbw, const float* ad,
                          const int8_t* aq, const int16_t* bs) {
    const uint8_t* hdr = w;
    const uint8_t* qsall = w + nbw * 16;
    float sums[8] = {0};
    float sumf = 0.f;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* h = hdr + (wb0 + b) * 16;
        const uint8_t* q4 = qsall + (wb0 + b) * 128;
        int8_t aux8[256];
        for (int j = 0; j < 4; j++) {
            for (int l = 0; l < 32; l++) aux8[64 * j + l] = (int8_t)(q4[32 * j + l] & 0xF);
            for (int l = 0; l < 32; l++) aux8[64 * j + 32 + l] = (int8_t)(q4[32 * j + l] >> 4);
        }
        uint8_t scales[8], mins[8];
        for (int j = 0; j < 8; j++) scale_min_k4(j, h + 4, &scales[j], &mins[j]);
        int sumi = 0;
        for (int j = 0; j < 16; j++) sumi += bs[b * 16 + j] * mins[j / 2];
        int aux32[8] = {0};
        const int8_t* a = aux8;
        const int8_t* q8 = aq + (size_t)b * 256;
        for (int j = 0; j < 8; j++) {
            int scale = scales[j];
            for (int t = 0; t < 4; t++) {
                for (int l = 0; l < 8; l++) aux32[l] += scale * (q8[l] * a[l]);
                q8 += 8;
                a += 8;
            }
        }
        uint16_t dh, mh;
        memcpy(&dh, h, 2);
        memcpy(&mh, h + 2, 2);
        float d = orc_f16_to_f32(dh) * ad[b];
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
        float dmin = orc_f16_to_f32(mh) * ad[b];
        sumf -= dmin * (float)sumi;
    }
    float t = 0.f;
    for (int l = 0; l < 8; l++) t += sums[l];
    return sumf + t;
}

typedef struct {
    int qt, M, N, K, n0, n1;
    const uint8_t* w;
    float* y;
    const uint8_t* a8;    /* q8_0 activations SoA, one per row (stride bytes) */
    size_t a8_stride;
    const float* kd;      /* q8_k */
    const int8_t* kq;
    const int16_t* kb;
} qmm_job;

static void* qmm_worker(void* p) {
    qmm_job* j = (qmm_job*)p;
    int K = j->K;
    size_t nbw = (size_t)j->N * K / (j->qt == ORC_Q4_K ? 256 : 32);
    for (int m = 0; m < j->M; m++) {
        for (int n = j->n0; n < j->n1; n++) {
            float r;
            if (j->qt == ORC_Q4_0)
                r = vec_dot_q4_0(K, j->w, (size_t)n * (K / 32), nbw, j->a8 + m * j->a8_stride, K / 32);
            else if (j->qt == ORC_Q8_0)
                r = vec_dot_q8_0(K, j->w, (size_t)n * (K / 32), nbw, j->a8 + m * j->a8_stride, K / 32);
            else
                r = vec_dot_q4_k(K, j->w, (size_t)n * (K / 256), nbw, j->kd + (size_t)m * (K / 256),
                                 j->kq + (size_t)m * K, j->kb + (size_t)m * (K / 16));
            j->y[(size_t)m * j->N + n] = r;
        }
    }
    return NULL;
}

/* y[M,N] = x[M,K] . W[N,K]^T with Candle's CPU method: each activation row is
 * quantized to the weight's vec-dot type (Q8_0 for Q4_0/Q8_0, Q8_K for Q4_K),
 * then every output is an integer block dot scaled per block. */
void orc_qmatmul(int qt, const uint8_t* w, const float* x, float* y, int M, int N, int K,
                 int nthreads) {
    if (nthreads < 1) nthreads = 1;
    uint8_t* a8 = NULL;
    float* kd = NULL;
    int8_t* kq = NULL;
    int16_t* kb = NULL;
    size_t a8_stride = (size_t)K / 32 * 34;
    if (qt == ORC_Q4_K) {
        kd = (float*)malloc(sizeof(float) * (size_t)M * (K / 256));
        kq = (int8_t*)malloc((size_t)M * K);
        kb = (int16_t*)malloc(sizeof(int16_t) * (size_t)M * (K / 16));
        for (int m = 0; m < M; m++)
            orc_quantize_q8_k(x + (size_t)m * K, K, kd + (size_t)m * (K / 256), kq + (size_t)m * K,
                              kb + (size_t)m * (K / 16));
    } else {
        a8 = (uint8_t*)malloc(a8_stride * M);
        for (int m = 0; m < M; m++) orc_quantize_q8_0(x + (size_t)m * K, K, a8 + m * a8_stride);
    }
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * nthreads);
    qmm_job* jobs = (qmm_job*)malloc(sizeof(qmm_job) * nthreads);
    int per = (N + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; t++) {
        qmm_job j = {qt, M, N, K, t * per, (t + 1) * per < N ? (t + 1) * per : N,
                     w, y, a8, a8_stride, kd, kq, kb};
        if (j.n0 > N) j.n0 = N;
        jobs[t] = j;
        if (nthreads > 1) pthread_create(&th[t], NULL, qmm_worker, &jobs[t]);
        else qmm_worker(&jobs[t]);
    }
    if (nthreads > 1)
        for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
    free(a8);
    free(kd);
    free(kq);
    free(kb);
}

/* ------------------------------------------------------------------ */
/* W8A16 / W4A16 GEMM                                                   */
/* ------------------------------------------------------------------ */

/* matmul_{bf16}_8bit (matmul.cpp:1186-1215 -> matmul_decoding.h:451-471):
 * the weight tile is dequantized in T, w = T(T(q) * scale[k/g, n]), then
 * MAC with f32 accumulation and one rounding to T.  group <= 0 -> per channel.
 * The accumulation here is f64 (a tighter reference than any f32 order). */
void orc_w8a16_gemm(const uint16_t* a, const int8_t* w, const uint16_t* sc, uint16_t* out,
                    int M, int K, int N, int group, int rhs_t) {
    if (group <= 0) group = K;
    float* wd = (float*)malloc(sizeof(float) * (size_t)K * N);
    for (int k = 0; k < K; k++)
        for (int n = 0; n < N; n++) {
            int8_t q = rhs_t ? w[(size_t)n * K + k] : w[(size_t)k * N + n];
            float s = orc_bf16_to_f32(sc[(size_t)(k / group) * N + n]);
            wd[(size_t)k * N + n] = orc_bf16_to_f32(orc_f32_to_bf16((float)q * s));
        }
    double* acc = (double*)malloc(sizeof(double) * N);
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) acc[n] = 0;
        for (int k = 0; k < K; k++) {
            double av = orc_bf16_to_f32(a[(size_t)m * K + k]);
            const float* wr = wd + (size_t)k * N;
            for (int n = 0; n < N; n++) acc[n] += av * wr[n];
        }
        for (int n = 0; n < N; n++) out[(size_t)m * N + n] = orc_f32_to_bf16((float)acc[n]);
    }
    free(acc);
    free(wd);
}

/* GPTQ-style W4 (the layout the north-star W4A16 config names):
 * q[k,n] = (qw[k/8, n] >> 4*(k%8)) & 15, z[g,n] = (qz[g, n/8] >> 4*(n%8)) & 15,
 * w = bf16((q - z) * s[g,n]) -- the integer difference is exact, the product of
 * a <=5-bit integer and a bf16 scale is exact in f32, so one rounding. */
void orc_w4a16_dequant(const int32_t* qw, const uint16_t* sc, const int32_t* qz, uint16_t* wout,
                       int K, int N, int group) {
    for (int k = 0; k < K; k++) {
        int g = k / group;
        for (int n = 0; n < N; n++) {
            int q = ((uint32_t)qw[(size_t)(k / 8) * N + n] >> (4 * (k % 8))) & 15;
            int z = ((uint32_t)qz[(size_t)g * (N / 8) + n / 8] >> (4 * (n % 8))) & 15;
            float s = orc_bf16_to_f32(sc[(size_t)g * N + n]);
            wout[(size_t)k * N + n] = orc_f32_to_bf16((float)(q - z) * s);
        }
    }
}

typedef struct {
    const uint16_t* a;
    const float* wd;
    uint16_t* out;
    int M, K, N, m0, m1;
} gemm_job;

static void* gemm_worker(void* p) {
    gemm_job* j = (gemm_job*)p;
    double* acc = (double*)malloc(sizeof(double) * j->N);
    for (int m = j->m0; m < j->m1; m++) {
        for (int n = 0; n < j->N; n++) acc[n] = 0;
        for (int k = 0; k < j->K; k++) {
            double av = orc_bf16_to_f32(j->a[(size_t)m * j->K + k]);
            const float* wr = j->wd + (size_t)k * j->N;
            for (int n = 0; n < j->N; n++) acc[n] += av * wr[n];
        }
        for (int n = 0; n < j->N; n++) j->out[(size_t)m * j->N + n] = orc_f32_to_bf16((float)acc[n]);
    }
    free(acc);
    return NULL;
}

static void gemm_bf16_f32w(const uint16_t* a, const float* wd, uint16_t* out, int M, int K, int N,
                           int nthreads) {
    if (nthreads < 1) nthreads = 1;
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * nthreads);
    gemm_job* jobs = (gemm_job*)malloc(sizeof(gemm_job) * nthreads);
    int per = (M + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; t++) {
        int m0 = t * per < M ? t * per : M, m1 = (t + 1) * per < M ? (t + 1) * per : M;
        gemm_job j = {a, wd, out, M, K, N, m0, m1};
        jobs[t] = j;
        if (nthreads > 1) pthread_create(&th[t], NULL, gemm_worker, &jobs[t]);
        else gemm_worker(&jobs[t]);
    }
    if (nthreads > 1)
        for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
}

void orc_w4a16_gemm(const uint16_t* a, const int32_t* qw, const uint16_t* sc, const int32_t* qz,
                    uint16_t* out, int M, int K, int N, int group, int nthreads) {
    uint16_t* wb = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)K * N);
    orc_w4a16_dequant(qw, sc, qz, wb, K, N, group);
    float* wd = (float*)malloc(sizeof(float) * (size_t)K * N);
    orc_bf16_to_f32_n(wb, wd, (size_t)K * N);
    free(wb);
    gemm_bf16_f32w(a, wd, out, M, K, N, nthreads);
    free(wd);
}

/* dequant_{f16,bf16} host lib (dequant_host.cpp:7-16): rhs u8 [K, N] holds
 * 2K weight rows, K being the *packed* row count; out [2K, N]; scale and zeros
 * T [2K/g, N].  The nibble order and zero rule live in the closed
 * acore::dequant (dequant_host.cpp:275) and are not pinned by any reference
 * test: restated as low nibble = row 2k, high nibble = row 2k+1,
 * w = T((q - zero) * scale) computed in f32. */
void orc_dequant_u4_ref(const uint8_t* rhs, const uint16_t* scale, const uint16_t* zeros,
                        uint16_t* out, int K, int N, int group, int dt) {
    int K2 = 2 * K;
    if (group <= 0) group = K2;
    for (int k = 0; k < K2; k++) {
        int g = k / group;
        for (int n = 0; n < N; n++) {
            uint8_t b = rhs[(size_t)(k / 2) * N + n];
            int q = (k & 1) ? (b >> 4) : (b & 15);
            float s = to_float_dt(scale, (size_t)g * N + n, dt);
            float z = to_float_dt(zeros, (size_t)g * N + n, dt);
            store_dt(out, (size_t)k * N + n, ((float)q - z) * s, dt);
        }
    }
}

/* ------------------------------------------------------------------ */
/* fp8 W8A8: out = bf16(sa[m] * sw[n] * sum_k a[m,k] w[k,n])             */
/* ------------------------------------------------------------------ */
typedef struct {
    const uint8_t* a;
    const float* sa;
    const float* wf;
    const float* sw;
    uint16_t* out;
    int M, K, N, m0, m1;
} fp8_job;

static void* fp8_worker(void* p) {
    fp8_job* j = (fp8_job*)p;
    double* acc = (double*)malloc(sizeof(double) * j->N);
    for (int m = j->m0; m < j->m1; m++) {
        for (int n = 0; n < j->N; n++) acc[n] = 0;
        for (int k = 0; k < j->K; k++) {
            double av = orc_e4m3_to_f32(j->a[(size_t)m * j->K + k]);
            if (av == 0) continue;
            const float* wr = j->wf + (size_t)k * j->N;
            for (int n = 0; n < j->N; n++) acc[n] += av * wr[n];
        }
        for (int n = 0; n < j->N; n++)
            j->out[(size_t)m * j->N + n] =
                orc_f32_to_bf16((float)(acc[n] * (double)j->sa[m] * (double)j->sw[n]));
    }
    free(acc);
    return NULL;
}

/* Per-row fp8 quantization (the activation / weight quantization the fp8
 * config names): scale = amax/448 (1 for an all-zero row), q = e4m3(x/scale). */
void orc_fp8_quantize_rows(const float* x, uint8_t* q, float* scale, int R, int C) {
    for (int r = 0; r < R; r++) {
        float amax = 0.f;
        for (int c = 0; c < C; c++) {
            float a = fabsf(x[(size_t)r * C + c]);
            if (a > amax) amax = a;
        }
        float s = amax > 0.f ? amax / 448.0f : 1.0f;
        scale[r] = s;
        for (int c = 0; c < C; c++) q[(size_t)r * C + c] = orc_f32_to_e4m3(x[(size_t)r * C + c] / s);
    }
}

void orc_fp8_gemm(const uint8_t* a, const float* sa, const uint8_t* w, const float* sw,
                  uint16_t* out, int M, int K, int N, int nthreads) {
    float lut[256];
    for (int i = 0; i < 256; i++) lut[i] = orc_e4m3_to_f32((uint8_t)i);
    float* wf = (float*)malloc(sizeof(float) * (size_t)K * N);
    for (size_t i = 0; i < (size_t)K * N; i++) wf[i] = lut[w[i]];
    if (nthreads < 1) nthreads = 1;
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * nthreads);
    fp8_job* jobs = (fp8_job*)malloc(sizeof(fp8_job) * nthreads);
    int per = (M + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; t++) {
        int m0 = t * per < M ? t * per : M, m1 = (t + 1) * per < M ? (t + 1) * per : M;
        fp8_job j = {a, sa, wf, sw, out, M, K, N, m0, m1};
        jobs[t] = j;
        if (nthreads > 1) pthread_create(&th[t], NULL, fp8_worker, &jobs[t]);
        else fp8_worker(&jobs[t]);
    }
    if (nthreads > 1)
        for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
    free(wf);
}

/* ------------------------------------------------------------------ */
/* MoE routing                                                          */
/* ------------------------------------------------------------------ */

/* topk_softmax_kernel_impl (topk_softmax_host.cpp:103-176): max-subtracted
 * softmax with expf, k rounds of arg-max over the probabilities (strict >, so
 * the lowest index wins a tie), outputs rounded to T; with norm the T-rounded
 * weights are scaled by 1/sum of the f32 probabilities picked. */
void orc_topk_softmax(const void* in, void* out, int32_t* idx, int T, int E, int k, int norm,
                      int dt) {
    float* prob = (float*)malloc(sizeof(float) * E);
    float* wtmp = (float*)malloc(sizeof(float) * E);
    for (int t = 0; t < T; t++) {
        size_t base = (size_t)t * E;
        float mx = -INFINITY;
        for (int e = 0; e < E; e++) {
            float v = to_float_dt(in, base + e, dt);
            if (v > mx) mx = v;
        }
        float sum = 0.f;
        for (int e = 0; e < E; e++) sum += expf(to_float_dt(in, base + e, dt) - mx);
        float inv = sum > 0.f ? 1.f / sum : 1.f;
        for (int e = 0; e < E; e++) prob[e] = expf(to_float_dt(in, base + e, dt) - mx) * inv;
        for (int e = 0; e < E; e++) wtmp[e] = prob[e];
        float wsum = 0.f;
        int got = 0;
        for (int j = 0; j < k; j++) {
            float best = -INFINITY;
            int bi = -1;
            for (int e = 0; e < E; e++)
                if (wtmp[e] > best) { best = wtmp[e]; bi = e; }
            if (bi < 0) break;
            store_dt(out, (size_t)t * k + j, prob[bi], dt);
            idx[(size_t)t * k + j] = bi;
            wsum += prob[bi];
            wtmp[bi] = -INFINITY;
            got++;
        }
        if (norm && wsum > 0.f) {
            float iv = 1.f / wsum;
            for (int j = 0; j < got; j++) {
                float v = to_float_dt(out, (size_t)t * k + j, dt) * iv;
                store_dt(out, (size_t)t * k + j, v, dt);
            }
        }
    }
    free(prob);
    free(wtmp);
}

/* moe_align_block_size (moe_align_host.cpp:587-764 scalar path, 766-921
 * kernel): flat slot i = t*k + j is bucketed by topk_ids[i] in ascending i;
 * each expert's run is padded to a multiple of bs with pad = T*k (the
 * original token count, moe_align_host.cpp:776); experts with no slot get no
 * block; experts_ids[blk] = expert (or expert_map[expert]); ntpp = sum of the
 * padded runs.  sorted_ids beyond ntpp hold the pad value and experts_ids
 * beyond the used blocks hold 0 (the memsets at :777-784).  real_token_num,
 * when given, limits the slots to real*k (:785-799).  Out-of-range ids trap in
 * the reference (check_ids, :101-163); here they return -1. */
int orc_moe_align_block_size(int32_t* sorted_ids, int32_t* experts_ids, int32_t* ntpp,
                             const int32_t* topk_ids, const int32_t* real_token_num,
                             const int32_t* expert_map, int E, int bs, int T, int k) {
    if (E <= 0 || bs <= 0 || T < 0 || k <= 0) return -1;
    int pad = T * k;
    int max_padded = T * k + E * (bs - 1);
    int max_blocks = max_padded / bs;
    for (int i = 0; i < max_padded; i++) sorted_ids[i] = pad;
    for (int i = 0; i < max_blocks; i++) experts_ids[i] = 0;
    int tn = T;
    if (real_token_num) {
        if (*real_token_num < 0 || *real_token_num > T) return -1;
        tn = *real_token_num;
    }
    int n = tn * k;
    for (int i = 0; i < n; i++)
        if (topk_ids[i] < 0 || topk_ids[i] >= E) return -1;
    if (expert_map)
        for (int e = 0; e < E; e++)
            if (expert_map[e] < -1 || expert_map[e] >= E) return -1;
    int* cnt = (int*)calloc(E, sizeof(int));
    int* off = (int*)calloc(E + 1, sizeof(int));
    for (int i = 0; i < n; i++) cnt[topk_ids[i]]++;
    for (int e = 0; e < E; e++) off[e + 1] = off[e] + (cnt[e] + bs - 1) / bs * bs;
    int total = off[E];
    for (int e = 0; e < E; e++)
        for (int b = off[e] / bs; b < off[e + 1] / bs; b++)
            experts_ids[b] = expert_map ? expert_map[e] : e;
    int* fill = (int*)calloc(E, sizeof(int));
    for (int i = 0; i < n; i++) {
        int e = topk_ids[i];
        sorted_ids[off[e] + fill[e]++] = i;
    }
    *ntpp = total;
    free(cnt);
    free(off);
    free(fill);
    return total;
}

/* invoke_fused_moe (fused_moe_host.cpp:43-252 and _splitm :254-453): for each
 * sorted block b < ntpp/bs with expert e:
 *   e == -1 -> rows C[s,:] = 0 for the valid slots s (stop at the first pad);
 *   else    -> C[s,n] = T(acc), acc = sum_k A[s/topk_str,k] * B[e,n,k] (+bias[e,n])
 *              and, with mul_routed_weight, acc *= topk_w[s] in f32 first.
 * topk_str = mul_routed_weight ? 1 : top_k (:84).  Slots s outside
 * [0, topk_ids_size) are skipped.  B is bf16 [E,N,K], or (Bq != NULL) int8
 * [E,N,K] with per-output-channel bf16 scales [E,N] applied to the f32
 * accumulator -- the W8A16 expert format that has no reference kernel. */
typedef struct {
    uint16_t* C;
    const uint16_t *A, *B, *Bs, *bias;
    const int8_t* Bq;
    const float* tw;
    const int32_t *sorted, *eids;
    int K, N, E, tis, top_k, bs, mrw, bias_flag, b0, b1;
} moe_job;

static void* moe_worker(void* p) {
    moe_job* j = (moe_job*)p;
    int topk_str = j->mrw ? 1 : j->top_k;
    int K = j->K, N = j->N;
    double* acc = (double*)malloc(sizeof(double) * N);
    float* arow = (float*)malloc(sizeof(float) * K);
    for (int b = j->b0; b < j->b1; b++) {
        int e = j->eids[b];
        for (int r = 0; r < j->bs; r++) {
            int s = j->sorted[b * j->bs + r];
            if (s < 0 || s >= j->tis) {
                if (e == -1) break;
                continue;
            }
            if (e == -1) {
                for (int n = 0; n < N; n++) j->C[(size_t)s * N + n] = 0;
                continue;
            }
            const uint16_t* ar = j->A + (size_t)(s / topk_str) * K;
            for (int kk = 0; kk < K; kk++) arow[kk] = orc_bf16_to_f32(ar[kk]);
            for (int n = 0; n < N; n++) {
                double a = 0;
                size_t wo = ((size_t)e * N + n) * K;
                if (j->Bq) {
                    for (int kk = 0; kk < K; kk++) a += (double)arow[kk] * (double)j->Bq[wo + kk];
                    a *= (double)orc_bf16_to_f32(j->Bs[(size_t)e * N + n]);
                } else {
                    for (int kk = 0; kk < K; kk++)
                        a += (double)arow[kk] * (double)orc_bf16_to_f32(j->B[wo + kk]);
                }
                acc[n] = a;
            }
            for (int n = 0; n < N; n++) {
                float v = (float)acc[n];
                if (j->bias_flag) v = v + orc_bf16_to_f32(j->bias[(size_t)e * N + n]);
                if (j->mrw) v = v * j->tw[s];
                j->C[(size_t)s * N + n] = orc_f32_to_bf16(v);
            }
        }
    }
    free(acc);
    free(arow);
    return NULL;
}

void orc_fused_moe(uint16_t* C, const uint16_t* A, const uint16_t* B, const int8_t* Bq,
                   const uint16_t* Bs, const uint16_t* bias, const float* tw,
                   const int32_t* sorted, const int32_t* eids, const int32_t* ntpp, int M, int K,
                   int N, int E, int tis, int top_k, int bs, int mrw, int bias_flag,
                   int nthreads) {
    (void)M;
    (void)E;
    int nblk = *ntpp / bs;
    if (*ntpp == 0) return;
    if (nthreads < 1) nthreads = 1;
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * nthreads);
    moe_job* jobs = (moe_job*)malloc(sizeof(moe_job) * nthreads);
    int per = (nblk + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; t++) {
        int b0 = t * per < nblk ? t * per : nblk, b1 = (t + 1) * per < nblk ? (t + 1) * per : nblk;
        moe_job j = {C, A, B, Bs, bias, Bq, tw, sorted, eids, K, N, E, tis, top_k, bs, mrw,
                     bias_flag, b0, b1};
        jobs[t] = j;
        if (nthreads > 1) pthread_create(&th[t], NULL, moe_worker, &jobs[t]);
        else moe_worker(&jobs[t]);
    }
    if (nthreads > 1)
        for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
}

/* ------------------------------------------------------------------ */
/* legacy MoE combine and indexed expert matmul (moe_host.cpp)          */
/* ------------------------------------------------------------------ */
static inline float tof_dt(int dt, uint16_t v) {
    return dt == 1 ? orc_f16_to_f32(v) : orc_bf16_to_f32(v);
}
static inline uint16_t fromf_dt(int dt, float v) {
    return dt == 1 ? orc_f32_to_f16(v) : orc_f32_to_bf16(v);
}

/* moe_host.cpp:57-76: one slot k at a time (the reference's per-SIP loop):
 * tmp = T(e * w1) (mul<T,T,float>), y = T(y + tmp) (add). */
void orc_moe_combine(int dt, uint16_t* y, const uint16_t* e_out, const float* w,
                     const uint32_t* idx, const uint32_t* top, int N, int K, int M, int topk) {
    for (int k = 0; k < K; k++) {
        if (idx[k] >= (uint32_t)N || top[k] >= (uint32_t)topk) continue;
        const float w1 = w[(size_t)idx[k] * topk + top[k]];
        uint16_t* yr = y + (size_t)idx[k] * M;
        const uint16_t* er = e_out + (size_t)k * M;
        for (int c = 0; c < M; c++) {
            const float tmp = tof_dt(dt, fromf_dt(dt, tof_dt(dt, er[c]) * w1));
            yr[c] = fromf_dt(dt, tof_dt(dt, yr[c]) + tmp);
        }
    }
}

/* moe_host.cpp:160-180 (batch > 12) and :237-270 (decode): the input row is
 * in[b, 0] when M == 1, else in[b, i] (:168, :247); the sum follows the
 * reference's own CPU check moe_matmul (:325-355). */
void orc_indexed_moe(int dt, const uint16_t* in, const uint16_t* w, uint16_t* out,
                     const uint32_t* idx, int N, int K, int M, int batch, int topk, int E) {
    for (int b = 0; b < batch; b++)
        for (int i = 0; i < topk; i++) {
            const uint32_t e = idx[(size_t)b * topk + i];
            if (e >= (uint32_t)E) continue;
            const uint16_t* xr = in + ((size_t)b * M + (M == 1 ? 0 : i)) * K;
            uint16_t* orow = out + ((size_t)b * topk + i) * N;
            for (int n = 0; n < N; n++) {
                const uint16_t* wr = w + ((size_t)e * N + n) * K;
                float a = 0.0f; /* moe_matmul (:339-346): f32, k in order, no fma */
                for (int k = 0; k < K; k++) a += tof_dt(dt, xr[k]) * tof_dt(dt, wr[k]);
                orow[n] = fromf_dt(dt, a);
            }
        }
}
