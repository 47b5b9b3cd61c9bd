/*
 * q4k_oracle.c -- plain-C CPU oracle for the Q4_K GEMM core.  TEST INFRASTRUCTURE ONLY.
 *
 * Loaded (via ctypes) only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg, as the checker or as the timed CPU baseline.  The product library never links it.
 *
 * A second, independent restatement (beside oracle/q4k_oracle.py) of:
 *   tools/q4k_ref.py:27-37    get_scale_min_k4
 *   tools/q4k_ref.py:39-61    dequantize_block_q4_K     (w = f32(f32(d*sc)*q) - f32(dmin*m))
 *   tools/q4k_ref.py:105-124  dequantize_block_q6_K     (w = f32(f32(d*sc[p>>4])*(code-32)))
 *   tools/q4k_ref.py:126-129  dequantize_block_q8_0     (w = f32(d*qs))
 *   tools/q4k_ref.py:76-84    bf16_round                (RNE; inf/nan truncated)
 *   tools/q4k_ref.py:86-92    matmul_q4k_col            (sequential fp32 MAC in K order)
 *   tools/glm_model_q4k_ref.py:96-116,214-299  fp32_rsqrt, glm_sigmoid, glm_silu
 *   tools/glm_model_q4k_ref.py:476-486        matmul_bf16_dot (7-way interleave + tree)
 *   tools/glm_model_q4k_ref.py:138-148,826-834 bf16_gt argmax of the LM head
 *
 * Build: gcc -O2 -ffp-contract=off (every float op is one correctly rounded binary32
 * op on x86-64 SSE; contraction off keeps mul and add separate).  See oracle/Makefile.
 */
#include <stdint.h>
#include <string.h>

#define QK_K 256

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Exact IEEE half -> single (subnormals normalised, inf/nan kept, payload widened). */
float oq_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1F, m = h & 0x3FF;
    if (e == 0) {
        if (m == 0) return u2f(s);
        int sh = 0;
        while (!(m & 0x400)) { m <<= 1; sh++; }
        return u2f(s | ((uint32_t)(113 - sh) << 23) | ((m & 0x3FF) << 13));
    }
    if (e == 31) return u2f(s | 0x7F800000u | (m << 13));
    return u2f(s | ((e + 112) << 23) | (m << 13));
}

uint16_t oq_bf16_round(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)(u >> 16);
    uint64_t r = (uint64_t)u + 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)((r & 0xFFFF0000u) >> 16);
}

static inline float bf2f(uint16_t b) { return u2f((uint32_t)b << 16); }

void oq_scale_min_k4(int j, const uint8_t* q, int* sc, int* m) {
    if (j < 4) { *sc = q[j] & 63; *m = q[j + 4] & 63; }
    else {
        *sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        *m  = (q[j + 4] >> 4)  | ((q[j] >> 6) << 4);
    }
}

static void deq_q4k_block(const uint8_t* b, float* y) {
    float d = oq_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    float dm = oq_f16_to_f32((uint16_t)(b[2] | (b[3] << 8)));
    const uint8_t* sc = b + 4;
    const uint8_t* qs = b + 16;
    for (int g = 0; g < 4; g++) {
        int s0, m0, s1, m1;
        oq_scale_min_k4(2 * g, sc, &s0, &m0);
        oq_scale_min_k4(2 * g + 1, sc, &s1, &m1);
        float d1 = d * (float)s0, mm1 = dm * (float)m0;
        float d2 = d * (float)s1, mm2 = dm * (float)m1;
        for (int l = 0; l < 32; l++) {
            float p = d1 * (float)(qs[32 * g + l] & 0xF);
            y[64 * g + l] = p - mm1;
        }
        for (int l = 0; l < 32; l++) {
            float p = d2 * (float)(qs[32 * g + l] >> 4);
            y[64 * g + 32 + l] = p - mm2;
        }
    }
}

static void deq_q6k_block(const uint8_t* b, float* y) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    float d = oq_f16_to_f32((uint16_t)(b[208] | (b[209] << 8)));
    for (int h = 0; h < 2; h++) {
        for (int l = 0; l < 32; l++) {
            int qhv = qh[32 * h + l];
            int c[4];
            c[0] = ((ql[64 * h + l] & 0xF) | (((qhv >> 0) & 3) << 4)) - 32;
            c[1] = ((ql[64 * h + l + 32] & 0xF) | (((qhv >> 2) & 3) << 4)) - 32;
            c[2] = ((ql[64 * h + l] >> 4) | (((qhv >> 4) & 3) << 4)) - 32;
            c[3] = ((ql[64 * h + l + 32] >> 4) | (((qhv >> 6) & 3) << 4)) - 32;
            for (int t = 0; t < 4; t++) {
                float ds = d * (float)sc[8 * h + l / 16 + 2 * t];
                y[128 * h + 32 * t + l] = ds * (float)c[t];
            }
        }
    }
}

static void deq_q8_0_block(const uint8_t* b, float* y) {
    float d = oq_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    for (int i = 0; i < 32; i++) y[i] = d * (float)(int8_t)b[2 + i];
}

enum { OQ_F16 = 1, OQ_Q8_0 = 8, OQ_Q4_K = 12, OQ_Q6_K = 14, OQ_BF16 = 30 };

static int type_geom(int t, int* qk, int* bs) {
    switch (t) {
        case OQ_Q4_K: *qk = 256; *bs = 144; return 0;
        case OQ_Q6_K: *qk = 256; *bs = 210; return 0;
        case OQ_Q8_0: *qk = 32; *bs = 34; return 0;
        case OQ_F16: *qk = 1; *bs = 2; return 0;
        case OQ_BF16: *qk = 1; *bs = 2; return 0;
        default: return -1;
    }
}

/* Dequantize n_weights (a whole number of blocks) into out.  Returns 0 or -1. */
int oq_dequant(int type, const uint8_t* raw, int64_t n_weights, float* out) {
    int qk, bs;
    if (type_geom(type, &qk, &bs) || n_weights % qk) return -1;
    int64_t nb = n_weights / qk;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t* b = raw + i * bs;
        float* y = out + i * qk;
        switch (type) {
            case OQ_Q4_K: deq_q4k_block(b, y); break;
            case OQ_Q6_K: deq_q6k_block(b, y); break;
            case OQ_Q8_0: deq_q8_0_block(b, y); break;
            case OQ_F16: y[0] = oq_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); break;
            case OQ_BF16: y[0] = bf2f((uint16_t)(b[0] | (b[1] << 8))); break;
        }
    }
    return 0;
}

/*
 * Reference-order GEMV straight from ggml rows: for each output n the row is dequantized
 * into a K-float scratch row, then for each activation row m
 * acc = f32(acc + f32(a[m][k] * w[k])) for k = 0..K-1, bf16 out.
 * scratch must hold K floats.  acc (nullable) receives the fp32 accumulators [M][N].
 * Rows [n0, n1) only (lets the caller time a subsample).
 */
int oq_gemv_ref(int type, const uint8_t* raw, int64_t N, int64_t K, const uint16_t* x,
                int64_t M, int64_t n0, int64_t n1, float* scratch, float* acc, uint16_t* y) {
    int qk, bs;
    if (type_geom(type, &qk, &bs) || K % qk || n0 < 0 || n1 > N || n0 > n1) return -1;
    int64_t rb = K / qk * bs;
    for (int64_t n = n0; n < n1; n++) {
        if (oq_dequant(type, raw + n * rb, K, scratch)) return -1;
        for (int64_t m = 0; m < M; m++) {
            const uint16_t* a = x + m * K;
            float s = 0.0f;
            for (int64_t k = 0; k < K; k++) {
                float p = bf2f(a[k]) * scratch[k];
                s = s + p;
            }
            if (acc) acc[m * N + n] = s;
            y[m * N + n] = oq_bf16_round(s);
        }
    }
    return 0;
}

/* ---- glm_model_q4k_ref.py:96-116 fp32_rsqrt ---- */
float oq_rsqrt(float x) {
    uint32_t u = f2u(x), e = (u >> 23) & 0xFF, man = u & 0x7FFFFF;
    if ((e == 0xFF && man) || (u >> 31) || e == 0) return u2f(0x7FC00000u);
    if (e == 0xFF) return 0.0f;
    float xh = 0.5f * x;
    float y = u2f(0x5F3759DFu - (u >> 1));
    for (int i = 0; i < 2; i++) {
        float yy = y * y;
        float xyy = xh * yy;
        float t = 1.5f - xyy;
        y = y * t;
    }
    return y;
}

/* ---- glm_model_q4k_ref.py:214-291 sigmoid core ---- */
static int round_half_up_int(float f) {
    uint32_t u = f2u(f), s = u >> 31, e = (u >> 23) & 0xFF, m = 0x800000u | (u & 0x7FFFFF);
    int r;
    if (e < 127) r = (e == 126) ? 1 : 0;
    else {
        int sh = 23 - ((int)e - 127);
        r = (int)((m >> sh) & 0xFF) + (int)((m >> (sh - 1)) & 1);
    }
    return s ? -r : r;
}

static float sanitize16(float x) {
    uint32_t u = f2u(x);
    if (((u >> 23) & 0xFF) == 0xFF) return u2f((u & 0x80000000u) | 0x41800000u);
    return x;
}

float oq_sigmoid_f32(float x) {
    float xs = sanitize16(x);
    uint32_t u = f2u(xs);
    if ((u & 0x7FFFFFFFu) >= 0x41800000u) xs = u2f((u & 0x80000000u) | 0x41800000u);
    float z = u2f(f2u(xs) ^ 0x80000000u);
    float kf = z * u2f(0x3FB8AA3Bu);
    int k = round_half_up_int(kf);
    if (k > 64) k = 64;
    if (k < -64) k = -64;
    float kl = (float)k * u2f(0x3F317218u);
    float r = z - kl;
    float p = u2f(0x3D2AAAABu) + r * u2f(0x3C088889u);
    p = u2f(0x3E2AAAABu) + r * p;
    p = u2f(0x3F000000u) + r * p;
    p = 1.0f + r * p;
    p = 1.0f + r * p;
    uint32_t pu = f2u(p);
    int en = (int)((pu >> 23) & 0xFF) + k;
    uint32_t sg = pu & 0x80000000u, ex;
    if (en >= 255) ex = sg | (0xFEu << 23) | (pu & 0x7FFFFF);
    else if (en <= 0) ex = sg;
    else ex = sg | ((uint32_t)en << 23) | (pu & 0x7FFFFF);
    float d = 1.0f + u2f(ex);
    float t = oq_rsqrt(d);
    return t * t;
}

uint16_t oq_glm_sigmoid(uint16_t xb) { return oq_bf16_round(oq_sigmoid_f32(bf2f(xb))); }

uint16_t oq_glm_silu(uint16_t xb) {
    float x = bf2f(xb);
    float s = oq_sigmoid_f32(x);
    return oq_bf16_round(s * sanitize16(x));
}

/* Bit-pattern wrappers (callers that marshal floats through doubles would quiet sNaNs). */
uint16_t oq_bf16_round_bits(uint32_t u) { return oq_bf16_round(u2f(u)); }
uint32_t oq_rsqrt_bits(uint32_t u) { return f2u(oq_rsqrt(u2f(u))); }
uint32_t oq_f16_to_f32_bits(uint16_t h) { return f2u(oq_f16_to_f32(h)); }

/* ---- glm_model_q4k_ref.py:476-486 matmul_bf16_dot: product k goes into partial sum
 * ps[k % 7] (ps starts at +0), then ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+0)), bf16 out. ---- */
uint16_t oq_bf16_dot7(const uint16_t* a, const uint16_t* w, int64_t K, float* sum_out) {
    float ps[7] = {0, 0, 0, 0, 0, 0, 0};
    for (int64_t k = 0; k < K; k++) {
        float prod = bf2f(a[k]) * bf2f(w[k]);
        ps[k % 7] = ps[k % 7] + prod;
    }
    float a01 = ps[0] + ps[1], a23 = ps[2] + ps[3], a45 = ps[4] + ps[5], a6 = ps[6] + 0.0f;
    float b0 = a01 + a23, b1 = a45 + a6;
    float s = b0 + b1;
    if (sum_out) *sum_out = s;
    return oq_bf16_round(s);
}

/* ---- glm_model_q4k_ref.py:138-148 bf16_gt: strict '>' on bf16 patterns ---- */
int oq_bf16_gt(uint16_t a, uint16_t b) {
    int sa = (a >> 15) & 1, sb = (b >> 15) & 1;
    int ma = a & 0x7FFF, mb = b & 0x7FFF;
    if (sa != sb) {
        if (ma == 0 && mb == 0) return 0;
        return sb == 1;
    }
    if (sa == 0) return ma > mb;
    return ma < mb;
}

/* ---- glm_model_q4k_ref.py:826-834: logits over rows [v0, v1) of the V x K bf16 head, and
 * the argmax scan (start at -inf = 0xFF80, index 0; replace only on strict bf16_gt).
 * argmax (nullable) is only meaningful for the full range v0 = 0, v1 = V. ---- */
int oq_lm_head(const uint16_t* w, int64_t V, int64_t K, const uint16_t* x, int64_t v0, int64_t v1,
               uint16_t* logits, int32_t* argmax) {
    if (v0 < 0 || v1 > V || v0 > v1 || K < 1) return -1;
    uint16_t best = 0xFF80;
    int32_t arg = 0;
    for (int64_t v = v0; v < v1; v++) {
        uint16_t lb = oq_bf16_dot7(x, w + v * K, K, 0);
        logits[v] = lb;
        if (oq_bf16_gt(lb, best)) {
            best = lb;
            arg = (int32_t)v;
        }
    }
    if (argmax) *argmax = arg;
    return 0;
}
