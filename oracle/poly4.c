/* Independent C restatement of the reference's poly4 GELU, used by the tests
 * to pin the numpy oracle (oracle/rowops.py gelu_poly4): two restatements
 * written from different primitives must agree bit for bit.
 *
 * TEST INFRASTRUCTURE ONLY -- not part of the product.
 *
 * Follows kernels/gelu_poly4_eval.inc:27-65 with the constants of
 * kernels/gelu_poly4_coeffs.h:4-13, the fp32 input rounding of
 * kernels/gelu_row4f.cc:58-84 (g4f) and the RNE / truncation modes of
 * kernels/gelu_row4_rne.cc:44-66 (g4r) and kernels/gelu_row4.cc:44-61 (g4).
 * Built with -ffp-contract=off so every fp32 operation rounds once, in the
 * order written.
 */
#include <stdint.h>
#include <string.h>

static const float BRK[3] = {1.0f, 2.0f, 4.0f};
static const float SHF[3] = {0.5f, 1.5f, 3.0f};
static const float SCL[3] = {2.0f, 2.0f, 1.0f};
static const float COEF[3][5] = {
    {-0.0020446777f, -0.013000488f, 0.077148438f, -0.06640625f, -0.15429688f},
    {0.0021514893f, -0.0071716309f, -0.0040283203f, 0.063964844f, -0.10009766f},
    {-0.0029296875f, 0.010681152f, -0.015869141f, 0.012023926f, -0.0040283203f},
};

static uint32_t bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* fp32 -> bf16 bits; mode 0 = round to nearest even, 1 = truncate */
static uint16_t to_bf16(float f, int mode) {
  uint32_t u = bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  if (mode == 1) return (uint16_t)(u >> 16);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static float rb(float f, int mode) { return from_bits((uint32_t)to_bf16(f, mode) << 16); }

/* x: n fp32 inputs (bf16-exact unless f32_input); y: n bf16 outputs */
void poly4_gelu(const float* x, uint16_t* y, long n, int mode, int f32_input) {
  for (long i = 0; i < n; ++i) {
    float xv = f32_input ? rb(x[i], 0) : x[i];
    float s = xv < 0.0f ? -xv : xv;
    float q = 0.0f;
    for (int p = 2; p >= 0; --p) {
      float t = rb(s - SHF[p], mode);
      float u = rb(t * SCL[p], mode);
      float acc = COEF[p][0];
      for (int k = 1; k <= 4; ++k) {
        float ah = rb(acc, mode);
        float prod = ah * u; /* exact: two bf16 factors */
        acc = COEF[p][k] + prod;
      }
      if (s < BRK[p]) q = rb(acc, mode);
    }
    float relu = xv > 0.0f ? xv : 0.0f;
    y[i] = to_bf16(relu + q, mode);
  }
}
