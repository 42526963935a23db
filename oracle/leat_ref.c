/* C restatement of leat's LEAT_KERNELS=ref linear layer: y = x @ dequant(W).T with unquantized
 * f32 activations and f32 accumulation (leat/ops.py:35-38, dequantization leat/quant.py:117-119,
 * 182-197, 213-223 in ggml's float operation order). Test infrastructure and the timed CPU
 * baseline only; the product never links it.
 *
 * Built with -ffp-contract=off so that d1 * q - m1 rounds twice, as ggml and gguf-py do; the
 * dequantized rows therefore equal oracle/leat_oracle.py's bit for bit (checked in tests).
 * The dot product keeps 8 partial sums (element i into sum i % 8) and adds them pairwise, a
 * fixed order the compiler can vectorise.
 */
#include <stdint.h>
#include <string.h>

enum { Q8_0 = 8, Q4_K = 12, Q6_K = 14 };

static float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float f16_at(const uint8_t *p) { return half_to_float((uint16_t)(p[0] | (p[1] << 8))); }

static void scale_min_k4(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

static void block_q8_0(const uint8_t *b, float *y) {
    float d = f16_at(b);
    for (int i = 0; i < 32; i++) y[i] = d * (float)(int8_t)b[2 + i];
}

static void block_q4_k(const uint8_t *b, float *y) {
    float d = f16_at(b), dmin = f16_at(b + 2);
    const uint8_t *scales = b + 4, *q = b + 16;
    for (int j = 0; j < 4; j++) {
        int sc, m;
        scale_min_k4(2 * j, scales, &sc, &m);
        float d1 = d * (float)sc, m1 = dmin * (float)m;
        scale_min_k4(2 * j + 1, scales, &sc, &m);
        float d2 = d * (float)sc, m2 = dmin * (float)m;
        for (int l = 0; l < 32; l++) y[64 * j + l] = d1 * (float)(q[32 * j + l] & 0xF) - m1;
        for (int l = 0; l < 32; l++) y[64 * j + 32 + l] = d2 * (float)(q[32 * j + l] >> 4) - m2;
    }
}

static void block_q6_k(const uint8_t *b, float *y) {
    float d = f16_at(b + 208);
    for (int n = 0; n < 2; n++) {
        const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n;
        const int8_t *sc = (const int8_t *)(b + 192 + 8 * n);
        float *out = y + 128 * n;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            out[l] = d * (float)sc[is + 0] * (float)q1;
            out[l + 32] = d * (float)sc[is + 2] * (float)q2;
            out[l + 64] = d * (float)sc[is + 4] * (float)q3;
            out[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
    }
}

static int block_shape(int type, int *elements, int *bytes) {
    switch (type) {
    case Q8_0: *elements = 32; *bytes = 34; return 0;
    case Q4_K: *elements = 256; *bytes = 144; return 0;
    case Q6_K: *elements = 256; *bytes = 210; return 0;
    default: return -1;
    }
}

static void decode(int type, const uint8_t *b, float *y) {
    if (type == Q8_0) block_q8_0(b, y);
    else if (type == Q4_K) block_q4_k(b, y);
    else block_q6_k(b, y);
}

int leat_ref_dequant(int type, const uint8_t *blocks, int64_t n_blocks, float *out) {
    int el, by;
    if (block_shape(type, &el, &by)) return -1;
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n_blocks; i++) decode(type, blocks + i * by, out + i * el);
    return 0;
}

/* out[t * rows + r] = sum_c x[t * cols + c] * W[r, c], W decoded block by block. */
int leat_ref_linear(int type, const uint8_t *w, int64_t rows, int64_t cols, const float *x,
                    int tokens, float *out) {
    int el, by;
    if (block_shape(type, &el, &by) || cols % el || tokens < 1 || tokens > 64) return -1;
    int64_t per_row = cols / el;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        float y[256];
        float acc[64][8];
        for (int t = 0; t < tokens; t++)
            for (int i = 0; i < 8; i++) acc[t][i] = 0.0f;
        for (int64_t b = 0; b < per_row; b++) {
            decode(type, w + (r * per_row + b) * by, y);
            for (int t = 0; t < tokens; t++) {
                const float *xs = x + t * cols + b * el;
                for (int i = 0; i < el; i += 8)
                    for (int k = 0; k < 8; k++) acc[t][k] += y[i + k] * xs[i + k];
            }
        }
        for (int t = 0; t < tokens; t++) {
            float *a = acc[t];
            out[t * rows + r] = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
        }
    }
    return 0;
}

/* The OpenMP threads the functions above use (the CPU baseline times all cores, then one). */
#include <omp.h>
void leat_ref_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int leat_ref_max_threads(void) { return omp_get_max_threads(); }
