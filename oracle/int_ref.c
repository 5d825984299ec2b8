/*
 * Plain-C restatement of the integer and byte work on the TESM BitLinear path.
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never linked into
 * the product library.
 *
 * Reference = WANGLILIN360/tesm.
 *   activation codes  tesm_ssm/modules/tesm.py:206-209 (BitLinear.quantized_input)
 *   weight codes      tesm_ssm/modules/tesm.py:211-215 (BitLinear.quantized_weight)
 *   INT2 packing      tesm_ssm/utils/int2_quantization.py:21-93
 *                     (code = q + 1, k = 4j + i lives in bits 2i..2i+1 of byte j,
 *                      rows padded with code 1, i.e. value 0)
 *   accumulators      the exact integer dot product behind F.linear of the
 *                     dequantized operands (tesm.py:273-276)
 *
 * Float semantics follow torch on the CPU: every float32 op is one IEEE single
 * operation (build with -ffp-contract=off), `127 / t` is `reciprocal(t) * 127`,
 * `round` is round-half-to-even.  The bf16 variants round every intermediate
 * result to bfloat16 (round to nearest even), as torch does for bf16 tensors.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* float -> nearest-even bfloat16, returned as the float it represents */
static float round_bf16(float f) {
    uint32_t u = f32_to_bits(f);
    if ((u & 0x7f800000u) == 0x7f800000u) return f; /* inf / nan unchanged */
    u += 0x7fffu + ((u >> 16) & 1u);
    return bits_to_f32(u & 0xffff0000u);
}

float oracle_round_bf16(float f) { return round_bf16(f); }

static float bf16_bits_to_f32(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

static float clamp_code(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Per-row int8 codes and scale for float32 rows (tesm.py:206-209). */
void oracle_quant_act_f32(const float* x, int64_t M, int64_t K, float eps, int8_t* q, float* s) {
    for (int64_t m = 0; m < M; ++m) {
        const float* row = x + m * K;
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) { float a = fabsf(row[k]); if (a > amax) amax = a; }
        float d = amax < eps ? eps : amax;
        float sc = (1.0f / d) * 127.0f;
        s[m] = sc;
        for (int64_t k = 0; k < K; ++k) q[m * K + k] = (int8_t)clamp_code(rintf(row[k] * sc), -128.f, 127.f);
    }
}

/* Same for bf16 rows given as raw bf16 bit patterns; every op rounds to bf16. */
void oracle_quant_act_bf16(const uint16_t* x, int64_t M, int64_t K, float eps, int8_t* q, float* s) {
    float eps_b = round_bf16(eps);
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* row = x + m * K;
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) { float a = fabsf(bf16_bits_to_f32(row[k])); if (a > amax) amax = a; }
        float d = amax < eps_b ? eps_b : amax;
        float sc = round_bf16(round_bf16(1.0f / d) * 127.0f);
        s[m] = sc;
        for (int64_t k = 0; k < K; ++k) {
            float v = round_bf16(bf16_bits_to_f32(row[k]) * sc);
            q[m * K + k] = (int8_t)clamp_code(rintf(v), -128.f, 127.f);
        }
    }
}

/* Ternary weight codes given the per-tensor scale s_w (tesm.py:213-214). */
void oracle_weight_codes_f32(const float* w, int64_t n, float s_w, int8_t* codes) {
    for (int64_t i = 0; i < n; ++i) codes[i] = (int8_t)clamp_code(rintf(w[i] * s_w), -1.f, 1.f);
}

void oracle_weight_codes_bf16(const uint16_t* w, int64_t n, float s_w, int8_t* codes) {
    for (int64_t i = 0; i < n; ++i)
        codes[i] = (int8_t)clamp_code(rintf(round_bf16(bf16_bits_to_f32(w[i]) * s_w)), -1.f, 1.f);
}

/* Canonical INT2 packing of ternary codes (int2_quantization.py:36-58). */
void oracle_pack_i2(const int8_t* codes, int64_t N, int64_t K, uint8_t* packed) {
    int64_t kb = (K + 3) / 4;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t j = 0; j < kb; ++j) {
            unsigned byte = 0;
            for (int i = 0; i < 4; ++i) {
                int64_t k = 4 * j + i;
                unsigned c = k < K ? (unsigned)(codes[n * K + k] + 1) : 1u;
                byte |= (c & 3u) << (2 * i);
            }
            packed[n * kb + j] = (uint8_t)byte;
        }
}

/* Inverse of the packing (int2_quantization.py:68-93), codes in {-1,0,1}. */
void oracle_unpack_i2(const uint8_t* packed, int64_t N, int64_t K, int8_t* codes) {
    int64_t kb = (K + 3) / 4;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k)
            codes[n * K + k] = (int8_t)(((packed[n * kb + k / 4] >> (2 * (k % 4))) & 3) - 1);
}

/* acc[m][n] = sum_k q[m][k] * w[n][k], exact in int64 then checked into int32. */
int oracle_bitlinear_acc(const int8_t* q, const int8_t* wcodes, int64_t M, int64_t N, int64_t K, int32_t* acc) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            int64_t a = 0;
            const int8_t* xr = q + m * K;
            const int8_t* wr = wcodes + n * K;
            for (int64_t k = 0; k < K; ++k) a += (int64_t)xr[k] * wr[k];
            if (a > INT32_MAX || a < INT32_MIN) return 1;
            acc[m * N + n] = (int32_t)a;
        }
    return 0;
}
