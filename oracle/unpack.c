/* Scalar C restatement of the reference's block decoders.
 *
 * TEST INFRASTRUCTURE ONLY: part of the CPU oracle, built into oracle/_build/liboracle.so and loaded
 * by the tests as a second, independent restatement beside the numpy one (oracle/blocks.py). The
 * library never links it.
 *
 * Each function follows `unpack32` of strata_mlx/blocks.py:57-194 run by run, in float32 as the
 * Metal code computes (every product here is exact in float32); the dense types follow
 * strata_mlx/gguf.py:150-276. The codebooks come from the caller (the tests pass the grids that
 * oracle/grids.py decodes), so this file holds no table of its own except ggml's ksigns closed form.
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

static float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 31, man = h & 1023;
    float v;
    if (exp == 0) {
        v = ldexpf((float)man, -24);
    } else if (exp == 31) {
        v = man ? NAN : INFINITY;
    } else {
        v = ldexpf((float)(man | 1024), (int)exp - 25);
    }
    return sign ? -v : v;
}

static float half_at(const uint8_t* b) { return half_to_float((uint16_t)(b[0] | (b[1] << 8))); }
static uint32_t u16_at(const uint8_t* b) { return (uint32_t)b[0] | ((uint32_t)b[1] << 8); }
static uint32_t u32_at(const uint8_t* b) { return u16_at(b) | (u16_at(b + 2) << 16); }
static uint8_t ksign(uint32_t i) { return (uint8_t)(i | ((uint32_t)(__builtin_popcount(i) & 1) << 7)); }

static const int kv[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* blocks.py:49-53 */
static float q3k_scale(const uint8_t* s, uint32_t k) {
    uint32_t p = k % 4, word = k / 4;
    uint32_t low = word < 2 ? (s[4 * word + p] & 15u) : ((uint32_t)s[4 * (word - 2) + p] >> 4);
    return (float)((int)(low | ((((uint32_t)s[8 + p] >> (2 * word)) & 3u) << 4)) - 32);
}

/* the n-th run of 32 weights of a row of blocks; returns 0, or -1 for a kind it does not take */
static int unpack32(int kind, const uint8_t* row, uint32_t n, float* w, const uint8_t* grid) {
    switch (kind) {
    case 42: { /* Q2_0, blocks.py:58-68 */
        const uint8_t* b = row + (n / 2) * 18;
        const uint8_t* q = b + 2 + 8 * (n % 2);
        float d = half_at(b);
        for (uint32_t i = 0; i < 8; ++i)
            for (uint32_t j = 0; j < 4; ++j) w[4 * i + j] = d * ((float)((q[i] >> (2 * j)) & 3) - 1.0f);
        return 0;
    }
    case 20: { /* IQ4_NL, blocks.py:69-77 */
        const uint8_t* b = row + n * 18;
        float d = half_at(b);
        for (uint32_t i = 0; i < 16; ++i) {
            w[i] = d * (float)kv[b[2 + i] & 15];
            w[16 + i] = d * (float)kv[b[2 + i] >> 4];
        }
        return 0;
    }
    case 23: { /* IQ4_XS, blocks.py:78-88 */
        const uint8_t* b = row + (n / 8) * 136;
        uint32_t ib = n % 8;
        uint32_t ls = (((uint32_t)b[4 + ib / 2] >> (4 * (ib % 2))) & 15) | (((u16_at(b + 2) >> (2 * ib)) & 3) << 4);
        float d = half_at(b) * ((float)ls - 32.0f);
        const uint8_t* q = b + 8 + 16 * ib;
        for (uint32_t i = 0; i < 16; ++i) {
            w[i] = d * (float)kv[q[i] & 15];
            w[16 + i] = d * (float)kv[q[i] >> 4];
        }
        return 0;
    }
    case 21: { /* IQ3_S, blocks.py:89-102; grid (512, 4) */
        const uint8_t* b = row + (n / 8) * 110;
        uint32_t ib = n % 8;
        float d = half_at(b) * (float)(1 + 2 * (((uint32_t)b[106 + ib / 2] >> (4 * (ib % 2))) & 15));
        uint32_t high = b[66 + ib];
        for (uint32_t l = 0; l < 8; ++l) {
            const uint8_t* g = grid + 4 * ((uint32_t)b[2 + 8 * ib + l] | (((high >> l) & 1) << 8));
            uint32_t sign = (uint32_t)b[74 + 4 * ib + l / 2] >> (4 * (l % 2));
            for (uint32_t j = 0; j < 4; ++j) {
                float v = d * (float)g[j];
                w[4 * l + j] = ((sign >> j) & 1) ? -v : v;
            }
        }
        return 0;
    }
    case 18: { /* IQ3_XXS, blocks.py:103-116; grid (256, 4) */
        const uint8_t* b = row + (n / 8) * 98;
        uint32_t ib = n % 8;
        uint32_t aux = u32_at(b + 66 + 4 * ib);
        float d = half_at(b) * (0.5f + (float)(aux >> 28)) * 0.5f;
        for (uint32_t l = 0; l < 8; ++l) {
            const uint8_t* g = grid + 4 * (uint32_t)b[2 + 8 * ib + l];
            uint32_t sign = (uint32_t)ksign((aux >> (7 * (l / 2))) & 127) >> (4 * (l % 2));
            for (uint32_t j = 0; j < 4; ++j) {
                float v = d * (float)g[j];
                w[4 * l + j] = ((sign >> j) & 1) ? -v : v;
            }
        }
        return 0;
    }
    case 11: { /* Q3_K, blocks.py:164-175 */
        const uint8_t* b = row + (n / 8) * 110;
        uint32_t r = n % 8;
        const uint8_t* q = b + 32 + 32 * (r / 4);
        uint32_t shift = 2 * (r % 4);
        float d = half_at(b + 108);
        float s0 = d * q3k_scale(b + 96, 2 * r), s1 = d * q3k_scale(b + 96, 2 * r + 1);
        for (uint32_t i = 0; i < 32; ++i) {
            int v = (int)(((uint32_t)q[i] >> shift) & 3) - ((((uint32_t)b[i] >> r) & 1) ? 0 : 4);
            w[i] = (i < 16 ? s0 : s1) * (float)v;
        }
        return 0;
    }
    case 12: { /* Q4_K, gguf.py:174-179, 207-213: code * (d * sc) + -(dmin * mn), sub-block = run */
        const uint8_t* b = row + (n / 8) * 144;
        uint32_t s = n % 8;
        const uint8_t* p = b + 4;
        uint32_t sc = s < 4 ? (p[s] & 63u) : ((p[s + 4] & 15u) | (((uint32_t)p[s - 4] >> 6) << 4));
        uint32_t mn = s < 4 ? (p[s + 4] & 63u) : (((uint32_t)p[s + 4] >> 4) | (((uint32_t)p[s] >> 6) << 4));
        float scale = half_at(b) * (float)sc, bias = -(half_at(b + 2) * (float)mn);
        const uint8_t* q = b + 16 + 32 * (s / 2);
        for (uint32_t i = 0; i < 32; ++i) {
            uint32_t code = (s % 2) ? ((uint32_t)q[i] >> 4) : (q[i] & 15u);
            volatile float prod = (float)code * scale; /* as numpy: a product, then the add */
            w[i] = prod + bias;
        }
        return 0;
    }
    case 13: { /* Q5_K, gguf.py:207-218: Q4_K's form, the fifth code bit of weight i at bit s of qh[i] */
        const uint8_t* b = row + (n / 8) * 176;
        uint32_t s = n % 8;
        const uint8_t* p = b + 4;
        uint32_t sc = s < 4 ? (p[s] & 63u) : ((p[s + 4] & 15u) | (((uint32_t)p[s - 4] >> 6) << 4));
        uint32_t mn = s < 4 ? (p[s + 4] & 63u) : (((uint32_t)p[s + 4] >> 4) | (((uint32_t)p[s] >> 6) << 4));
        float scale = half_at(b) * (float)sc, bias = -(half_at(b + 2) * (float)mn);
        const uint8_t* qh = b + 16;
        const uint8_t* q = b + 48 + 32 * (s / 2);
        for (uint32_t i = 0; i < 32; ++i) {
            uint32_t code = ((s % 2) ? ((uint32_t)q[i] >> 4) : (q[i] & 15u)) | ((((uint32_t)qh[i] >> s) & 1u) << 4);
            volatile float prod = (float)code * scale;
            w[i] = prod + bias;
        }
        return 0;
    }
    case 14: { /* Q6_K, gguf.py:150-165 */
        const uint8_t* b = row + (n / 8) * 210;
        uint32_t r8 = n % 8, h = r8 / 4, r = r8 % 4;
        const uint8_t* ql = b + 64 * h;
        const uint8_t* qh = b + 128 + 32 * h;
        float d = half_at(b + 208);
        for (uint32_t i = 0; i < 32; ++i) {
            uint32_t lo = r == 0 ? (ql[i] & 15u) : r == 1 ? (ql[32 + i] & 15u) : r == 2 ? ((uint32_t)ql[i] >> 4)
                                                                                     : ((uint32_t)ql[32 + i] >> 4);
            uint32_t hi = ((uint32_t)qh[i] >> (2 * r)) & 3;
            int code = (int)(lo | (hi << 4)) - 32;
            uint32_t at = 128 * h + 32 * r + i;
            float scale = d * (float)(int8_t)b[192 + at / 16];
            w[i] = (float)code * scale;
        }
        return 0;
    }
    case 8: { /* Q8_0, gguf.py:203-206 */
        const uint8_t* b = row + n * 34;
        float d = half_at(b);
        for (uint32_t i = 0; i < 32; ++i) w[i] = d * (float)(int8_t)b[2 + i];
        return 0;
    }
    case 2: { /* Q4_0, gguf.py:195-197 */
        const uint8_t* b = row + n * 18;
        float d = half_at(b);
        for (uint32_t i = 0; i < 16; ++i) {
            w[i] = d * (float)((int)(b[2 + i] & 15) - 8);
            w[16 + i] = d * (float)((int)(b[2 + i] >> 4) - 8);
        }
        return 0;
    }
    case 6: { /* Q5_0, gguf.py:198-202 */
        const uint8_t* b = row + n * 22;
        float d = half_at(b);
        uint32_t qh = u32_at(b + 2);
        for (uint32_t i = 0; i < 16; ++i) {
            uint32_t lo = (b[6 + i] & 15u) | (((qh >> i) & 1) << 4);
            uint32_t hi = ((uint32_t)b[6 + i] >> 4) | (((qh >> (16 + i)) & 1) << 4);
            w[i] = d * (float)((int)lo - 16);
            w[16 + i] = d * (float)((int)hi - 16);
        }
        return 0;
    }
    default:
        return -1;
    }
}

/* every weight of `rows` rows of `cols` weights, rows of `row_bytes` bytes */
int oracle_dequant(int kind, const uint8_t* blocks, int64_t rows, int64_t cols, int64_t row_bytes,
                   const uint8_t* grid, float* out) {
    if (cols % 32) return -1;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t n = 0; n < cols / 32; ++n)
            if (unpack32(kind, blocks + r * row_bytes, (uint32_t)n, out + r * cols + 32 * n, grid)) return -1;
    return 0;
}

/* out[p, r] = sum over runs n, in order, of (sum over j of w[j] * x[j]) in float32, as _MATVEC does with one
   thread to a row (strata_mlx/blocks.py:196-220); x (pairs / share, cols) float32 */
int oracle_matvec(int kind, const uint8_t* blocks, int64_t rows, int64_t cols, int64_t row_bytes,
                  const uint32_t* idx, int64_t pairs, const float* x, int64_t share, const uint8_t* grid, float* out) {
    float w[32];
    for (int64_t p = 0; p < pairs; ++p)
        for (int64_t r = 0; r < rows; ++r) {
            const uint8_t* row = blocks + ((int64_t)idx[p] * rows + r) * row_bytes;
            const float* xr = x + (p / share) * cols;
            float sum = 0.0f;
            for (int64_t n = 0; n < cols / 32; ++n) {
                if (unpack32(kind, row, (uint32_t)n, w, grid)) return -1;
                float s = 0.0f;
                for (int j = 0; j < 32; ++j) s += w[j] * xr[32 * n + j];
                sum += s;
            }
            out[p * rows + r] = sum;
        }
    return 0;
}
