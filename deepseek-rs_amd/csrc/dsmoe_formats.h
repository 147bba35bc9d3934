// Block formats, lookup tables and scalar helpers shared by the HIP kernels
// (device) and the host library (host).  Everything here is plain C++ that
// compiles for both sides; nothing depends on torch.
//
// Formats (all little-endian, byte-packed, consumed exactly as the GGUF
// tensors store them):
//   IQ2_XXS  66 B / 256 weights : f16 d | u16 qs[32]
//            engine/src/kernels/quantize.rs:756-812, model.rs:31-83
//   Q2_K     84 B / 256 weights : u8 scales[16] | u8 qs[64] | f16 d | f16 dmin
//            engine/src/kernels/quantize.rs:840-901
//   Q8_K    292 B / 256 acts    : f32 d | i8 qs[256] | i16 bsums[16]
//            engine/src/kernels/quantize.rs:299-417
//   Q8_0     34 B / 32 weights  : f16 d | i8 qs[32]
//            engine/src/kernels/quantize.rs:147-225, matmul.rs:350-405
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define DSM_HD __host__ __device__ __forceinline__
#else
#define DSM_HD static inline
#endif

namespace dsm {

constexpr int QK_K = 256;
constexpr int QK8_0 = 32;
constexpr int IQ2XXS_BYTES = 66;
constexpr int Q2K_BYTES = 84;
constexpr int Q8K_BYTES = 292;
constexpr int Q8_0_BYTES = 34;

// IQ2_XXS codebook: 256 entries of 8 unsigned magnitudes, each byte one of
// {8, 25, 43}.  This is the fixed IQ2_XXS format table (the GGUF/ggml
// codebook); the values must be identical to
// engine/src/kernels/quantize.rs:431-688 for the bytes to decode the same.
#if defined(__HIPCC__)
__device__ __constant__
#endif
static const uint64_t kIq2xxsGrid[256] = {
    0x0808080808080808ull, 0x080808080808082bull, 0x0808080808081919ull, 0x0808080808082b08ull,
    0x0808080808082b2bull, 0x0808080808190819ull, 0x0808080808191908ull, 0x08080808082b0808ull,
    0x08080808082b082bull, 0x08080808082b2b08ull, 0x08080808082b2b2bull, 0x0808080819080819ull,
    0x0808080819081908ull, 0x0808080819190808ull, 0x0808080819192b08ull, 0x08080808192b0819ull,
    0x08080808192b1908ull, 0x080808082b080808ull, 0x080808082b08082bull, 0x080808082b082b2bull,
    0x080808082b2b082bull, 0x0808081908080819ull, 0x0808081908081908ull, 0x0808081908190808ull,
    0x0808081908191919ull, 0x0808081919080808ull, 0x080808192b081908ull, 0x080808192b192b08ull,
    0x0808082b08080808ull, 0x0808082b0808082bull, 0x0808082b082b082bull, 0x0808082b2b08082bull,
    0x0808190808080819ull, 0x0808190808081908ull, 0x0808190808190808ull, 0x08081908082b0819ull,
    0x08081908082b1908ull, 0x0808190819080808ull, 0x080819081908082bull, 0x0808190819082b08ull,
    0x08081908192b0808ull, 0x080819082b080819ull, 0x080819082b081908ull, 0x080819082b190808ull,
    0x080819082b2b1908ull, 0x0808191908080808ull, 0x080819190808082bull, 0x0808191908082b08ull,
    0x08081919082b0808ull, 0x080819191908192bull, 0x08081919192b2b19ull, 0x080819192b080808ull,
    0x080819192b190819ull, 0x0808192b08082b19ull, 0x0808192b08190808ull, 0x0808192b19080808ull,
    0x0808192b2b081908ull, 0x0808192b2b2b1908ull, 0x08082b0808080808ull, 0x08082b0808081919ull,
    0x08082b0808082b08ull, 0x08082b0808191908ull, 0x08082b08082b2b08ull, 0x08082b0819080819ull,
    0x08082b0819081908ull, 0x08082b0819190808ull, 0x08082b081919082bull, 0x08082b082b082b08ull,
    0x08082b1908081908ull, 0x08082b1919080808ull, 0x08082b2b0808082bull, 0x08082b2b08191908ull,
    0x0819080808080819ull, 0x0819080808081908ull, 0x0819080808190808ull, 0x08190808082b0819ull,
    0x0819080819080808ull, 0x08190808192b0808ull, 0x081908082b081908ull, 0x081908082b190808ull,
    0x081908082b191919ull, 0x0819081908080808ull, 0x0819081908082b08ull, 0x08190819082b0808ull,
    0x0819081919190808ull, 0x0819081919192b2bull, 0x081908192b080808ull, 0x0819082b082b1908ull,
    0x0819082b19081919ull, 0x0819190808080808ull, 0x0819190808082b08ull, 0x08191908082b0808ull,
    0x08191908082b1919ull, 0x0819190819082b19ull, 0x081919082b080808ull, 0x0819191908192b08ull,
    0x08191919192b082bull, 0x0819192b08080808ull, 0x0819192b0819192bull, 0x08192b0808080819ull,
    0x08192b0808081908ull, 0x08192b0808190808ull, 0x08192b0819080808ull, 0x08192b082b080819ull,
    0x08192b1908080808ull, 0x08192b1908081919ull, 0x08192b192b2b0808ull, 0x08192b2b19190819ull,
    0x082b080808080808ull, 0x082b08080808082bull, 0x082b080808082b2bull, 0x082b080819081908ull,
    0x082b0808192b0819ull, 0x082b08082b080808ull, 0x082b08082b08082bull, 0x082b0819082b2b19ull,
    0x082b081919082b08ull, 0x082b082b08080808ull, 0x082b082b0808082bull, 0x082b190808080819ull,
    0x082b190808081908ull, 0x082b190808190808ull, 0x082b190819080808ull, 0x082b19081919192bull,
    0x082b191908080808ull, 0x082b191919080819ull, 0x082b1919192b1908ull, 0x082b192b2b190808ull,
    0x082b2b0808082b08ull, 0x082b2b08082b0808ull, 0x082b2b082b191908ull, 0x082b2b2b19081908ull,
    0x1908080808080819ull, 0x1908080808081908ull, 0x1908080808190808ull, 0x1908080808192b08ull,
    0x19080808082b0819ull, 0x19080808082b1908ull, 0x1908080819080808ull, 0x1908080819082b08ull,
    0x190808081919192bull, 0x19080808192b0808ull, 0x190808082b080819ull, 0x190808082b081908ull,
    0x190808082b190808ull, 0x1908081908080808ull, 0x19080819082b0808ull, 0x19080819192b0819ull,
    0x190808192b080808ull, 0x190808192b081919ull, 0x1908082b08080819ull, 0x1908082b08190808ull,
    0x1908082b19082b08ull, 0x1908082b1919192bull, 0x1908082b192b2b08ull, 0x1908190808080808ull,
    0x1908190808082b08ull, 0x19081908082b0808ull, 0x190819082b080808ull, 0x190819082b192b19ull,
    0x190819190819082bull, 0x19081919082b1908ull, 0x1908192b08080808ull, 0x19082b0808080819ull,
    0x19082b0808081908ull, 0x19082b0808190808ull, 0x19082b0819080808ull, 0x19082b0819081919ull,
    0x19082b1908080808ull, 0x19082b1919192b08ull, 0x19082b19192b0819ull, 0x19082b192b08082bull,
    0x19082b2b19081919ull, 0x19082b2b2b190808ull, 0x1919080808080808ull, 0x1919080808082b08ull,
    0x1919080808190819ull, 0x1919080808192b19ull, 0x19190808082b0808ull, 0x191908082b080808ull,
    0x191908082b082b08ull, 0x1919081908081908ull, 0x191908191908082bull, 0x191908192b2b1908ull,
    0x1919082b2b190819ull, 0x191919082b190808ull, 0x191919082b19082bull, 0x1919191908082b2bull,
    0x1919192b08080819ull, 0x1919192b19191908ull, 0x19192b0808080808ull, 0x19192b0808190819ull,
    0x19192b0808192b19ull, 0x19192b08192b1908ull, 0x19192b1919080808ull, 0x19192b2b08082b08ull,
    0x192b080808081908ull, 0x192b080808190808ull, 0x192b080819080808ull, 0x192b0808192b2b08ull,
    0x192b081908080808ull, 0x192b081919191919ull, 0x192b082b08192b08ull, 0x192b082b192b0808ull,
    0x192b190808080808ull, 0x192b190808081919ull, 0x192b191908190808ull, 0x192b19190819082bull,
    0x192b19192b081908ull, 0x192b2b081908082bull, 0x2b08080808080808ull, 0x2b0808080808082bull,
    0x2b08080808082b2bull, 0x2b08080819080819ull, 0x2b0808082b08082bull, 0x2b08081908081908ull,
    0x2b08081908192b08ull, 0x2b08081919080808ull, 0x2b08082b08190819ull, 0x2b08190808080819ull,
    0x2b08190808081908ull, 0x2b08190808190808ull, 0x2b08190808191919ull, 0x2b08190819080808ull,
    0x2b081908192b0808ull, 0x2b08191908080808ull, 0x2b0819191908192bull, 0x2b0819192b191908ull,
    0x2b08192b08082b19ull, 0x2b08192b19080808ull, 0x2b08192b192b0808ull, 0x2b082b080808082bull,
    0x2b082b1908081908ull, 0x2b082b2b08190819ull, 0x2b19080808081908ull, 0x2b19080808190808ull,
    0x2b190808082b1908ull, 0x2b19080819080808ull, 0x2b1908082b2b0819ull, 0x2b1908190819192bull,
    0x2b1908192b080808ull, 0x2b19082b19081919ull, 0x2b19190808080808ull, 0x2b191908082b082bull,
    0x2b19190819081908ull, 0x2b19191919190819ull, 0x2b192b082b080819ull, 0x2b192b19082b0808ull,
    0x2b2b08080808082bull, 0x2b2b080819190808ull, 0x2b2b08082b081919ull, 0x2b2b081908082b19ull,
    0x2b2b082b08080808ull, 0x2b2b190808192b08ull, 0x2b2b2b0819190808ull, 0x2b2b2b1908081908ull,
};

// Sign byte for a 7-bit sign index: bit 7 restores even parity, which is
// what the 128-entry sign table of quantize.rs:693-701 tabulates.
DSM_HD uint32_t iq2_sign_byte(uint32_t idx7) {
  return idx7 | ((uint32_t)(__builtin_popcount(idx7) & 1) << 7);
}

// f16 bits -> f32 with subnormals flushed to zero, Inf/NaN kept
// (engine/src/kernels/utils.rs:16-29).
DSM_HD float f16_to_f32_ftz(uint16_t h) {
  uint32_t u = h;
  uint32_t sign = (u & 0x8000u) << 16;
  uint32_t ex = (u >> 10) & 0x1Fu;
  uint32_t man = u & 0x3FFu;
  uint32_t bits;
  if (ex == 0) bits = sign;
  else if (ex == 31) bits = sign | 0x7F800000u | (man << 13);
  else bits = sign | ((ex + 112u) << 23) | (man << 13);
  return __builtin_bit_cast(float, bits);
}
// s_setreg operand for MODE bits 7:6, the f16 / f64 denormal mode (hwreg
// id 1, offset 6, size 2).  With both bits clear the wave flushes f16 input
// denormals: the hardware widening then gives f16_to_f32_ftz's bits for
// every finite f16 value (a signalling NaN comes out quiet).  f32
// arithmetic keeps its own mode (bits 5:4).
constexpr int kHwregModeF16F64Denorm = 1 | (6 << 6) | ((2 - 1) << 11);
// The kernels' default for those bits: f16 / f64 denormals kept (in and out).
constexpr int kModeF16F64Preserve = 3;

// The same bits without branches (for loops that convert many values per
// step): exponent and mantissa move up 13 bits and the exponent is rebiased
// by 112 (<< 23 = 0x38000000), once more for Inf/NaN (31 -> 255), and
// exponent 0 (zero, subnormal) gives a signed zero.
DSM_HD float f16_to_f32_ftz_nb(uint16_t h) {
  const uint32_t u = h;
  const uint32_t sign = (u & 0x8000u) << 16;
  const uint32_t em = u & 0x7FFFu;
  uint32_t bits = (em << 13) + 0x38000000u;
  bits = em >= 0x7C00u ? bits + 0x38000000u : bits;
  bits = em < 0x0400u ? 0u : bits;
  return __builtin_bit_cast(float, sign | bits);
}

// f32 -> f16 bits, round to nearest even, with gradual underflow.  Used only
// by the synthetic-weight quantizers (the reference ships pre-quantized
// weights and has no encoder).
DSM_HD uint16_t f32_to_f16_rne(float f) {
  uint32_t x = __builtin_bit_cast(uint32_t, f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds to >= 65520 -> Inf
  if (ax < 0x33000001u) return (uint16_t)sign;               // < 2^-25 (+tie) -> 0
  uint32_t e = ax >> 23;
  uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
  if (e < 113) {  // subnormal half: value = m * 2^(e-150), unit 2^-24
    uint32_t shift = 126 - e;  // 14 .. 24
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t q = ((e - 112) << 10) | ((m >> 13) & 0x3FFu);
  uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
  return (uint16_t)(sign | q);
}

DSM_HD uint16_t ld_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
DSM_HD float ld_f32(const uint8_t* p) {
  uint32_t u = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
  return __builtin_bit_cast(float, u);
}

}  // namespace dsm
