// gfx950 kernels of the MoE-FFN path.  Built as a code object
// (hipcc --genco --offload-arch=gfx950) and loaded by dsmoe_host.cpp with
// hipModuleLoad; every kernel takes one argument struct from dsmoe_kargs.h.
//
// Memory layout in HBM is the GGUF layout the reference consumes:
//   gate/up  [E][I][d/256] IQ2_XXS blocks (66 B), row = d/256 blocks
//   down     [E][d][I/256] Q2_K blocks (84 B)
//   shared   [I_s][d/32] and [d][I_s/32] Q8_0 blocks (34 B)
//   router   [E][d] f16
// Weight rows are streamed with 16-byte vector loads over "block pairs":
// two IQ2_XXS blocks (132 B) or two Q8_0 blocks (68 B) always start on a
// 4-byte boundary even though a single block does not, so a pair is loaded
// as whole dwords and the odd-aligned block is re-aligned in registers.
// Per-block float results go to LDS and are summed per row in the
// reference's lane order (lane-strided partials, then a halving tree), which
// makes every row sum bit-identical to the reference arithmetic.
#include <hip/hip_runtime.h>

#include "dsmoe_formats.h"
#include "dsmoe_kargs.h"
#include "dsmoe_math.h"
#include "dsmoe_synth.h"

using namespace dsm;

namespace {

// Accesses to data that other workgroups of the same launch produce or
// consume (kCoh = true: the mid rows that dsmoe_up_rows quantizes in the
// workgroup completing a 256-row block) are agent-scope relaxed
// atomics: they compile to plain loads/stores with the device-coherence bit,
// which needs no L2 write-back or invalidate.  Ordering comes from waiting for
// the stores (s_waitcnt) before a counter is bumped.  With kCoh = false they
// are ordinary accesses (separate launches order everything).
template <bool kCoh, class T>
__device__ __forceinline__ T ldc(const T* p) {
  if constexpr (kCoh) return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else return *p;
}
template <bool kCoh, class T>
__device__ __forceinline__ void stc(T* p, T v) {
  if constexpr (kCoh) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}

constexpr int kQ8Stride = 272;  // LDS bytes per Q8_K block of qs (256 + pad)

__device__ __forceinline__ uint32_t alignbyte(uint32_t hi, uint32_t lo, uint32_t s) {
  return __builtin_amdgcn_alignbyte(hi, lo, s);
}

__device__ __forceinline__ int32_t dot4(uint32_t a, uint32_t b, int32_t c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ uint64_t sign_mask64(uint32_t sb) {
  uint64_t m = 0;
  for (int i = 0; i < 8; i++)
    if ((sb >> i) & 1u) m |= 0xFFull << (8 * i);
  return m;
}

struct Iq2Tables {
  uint64_t grid[256];
  uint64_t mask[128];  // byte-wise 0xFF where the element is negative
};

__device__ __forceinline__ void load_iq2_tables(Iq2Tables* t) {
  for (int i = threadIdx.x; i < 256; i += blockDim.x) t->grid[i] = kIq2xxsGrid[i];
  for (int i = threadIdx.x; i < 128; i += blockDim.x) t->mask[i] = sign_mask64(iq2_sign_byte(i));
}

// IQ2_XXS block . Q8_K block (qs in LDS) -> float (quantize.rs:763-812).
// `w` holds the 33 dwords of a 132-byte block pair; kSecond selects the block
// at byte 66 (its qs are dwords 17..32) instead of the block at byte 0 (qs
// start at byte 2, re-aligned here with alignbyte).
template <bool kSecond>
__device__ __forceinline__ uint32_t pair_qs(const uint32_t* w, int j) {
  return kSecond ? w[17 + j] : alignbyte(w[j + 1], w[j], 2);
}

template <bool kSecond>
__device__ __forceinline__ float iq2_block_dot(const uint32_t* w, const uint8_t* q8, float yd, const Iq2Tables* t) {
  int32_t bsum = 0;
#pragma unroll
  for (int ib = 0; ib < 8; ib++) {
    // z is an opaque zero that depends on the running sum: it keeps this
    // sub-block's LDS lookups after the previous sub-block's arithmetic.
    // Without it the compiler issues all 64 lookups of a block pair up front
    // and spills them.
    int z = 0;
    asm volatile("" : "+v"(z) : "v"(bsum));
    const uint32_t aux0 = pair_qs<kSecond>(w, 2 * ib) + z, aux1 = pair_qs<kSecond>(w, 2 * ib + 1) + z;
    const uint4 qa = *(const uint4*)(q8 + ib * 32 + z);
    const uint4 qb = *(const uint4*)(q8 + ib * 32 + 16 + z);
    // sum_i s_i g_i q_i = sum_i g_i q_i - 2 sum_i (g_i & m_i) q_i, m = 0xFF
    // on the negative elements: one AND per dword instead of a negation.
    // The grid operand stays unsigned here; variants that applied the signs
    // to the grid bytes before the dot failed parity and were not pursued.
    int32_t pos = 0, neg = 0;
    const uint32_t qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const uint64_t gv = t->grid[(aux0 >> (8 * g)) & 0xFF];
      const uint64_t mv = t->mask[(aux1 >> (7 * g)) & 127];
      pos = dot4((uint32_t)gv, qv[2 * g], pos);
      pos = dot4((uint32_t)(gv >> 32), qv[2 * g + 1], pos);
      neg = dot4((uint32_t)(gv & mv), qv[2 * g], neg);
      neg = dot4((uint32_t)((gv & mv) >> 32), qv[2 * g + 1], neg);
    }
    const int32_t ls = (int32_t)((aux1 >> 27) | 1u);  // 2 * (aux1 >> 28) + 1
    const int32_t sumi = pos - neg - neg;              // |sumi| <= 32*43*127 < 2^23
    bsum += __mul24(sumi, ls);  // |sumi| < 2^18, ls <= 31: one v_mad_i32_i24
  }
  const uint32_t dbits = kSecond ? (w[16] >> 16) : (w[0] & 0xFFFF);
  const float xd = f16_to_f32_ftz((uint16_t)dbits);
  return 0.125f * xd * yd * (float)bsum;
}

// Q2_K block (21 dwords) . Q8_K block -> float (quantize.rs:846-901).
__device__ __forceinline__ float q2k_block_dot(const uint32_t* w, const uint8_t* q8, const int16_t* bsums,
                                               float yd) {
  int32_t summs = 0;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const uint32_t sc = (w[j >> 2] >> (8 * (j & 3))) & 0xFF;
    summs += (int32_t)bsums[j] * (int32_t)(sc >> 4);
  }
  // The 2-bit field j of every byte is masked in place for j < 3 (values
  // c * 4^j <= 48 stay positive int8), so its group sums come out 4^j times
  // too large and are accumulated apart, then shifted back (exact: every
  // term is a multiple of 4^j).
  int32_t acc[4] = {0, 0, 0, 0};
#pragma unroll
  for (int k = 0; k < 2; k++) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int G = 8 * k + 2 * j + h;
        const uint32_t sc = (w[G >> 2] >> (8 * (G & 3))) & 0xF;
        int z = 0;  // opaque zero: keeps this group's LDS read after the previous group's sum
        asm volatile("" : "+v"(z) : "v"(acc[j]));
        const uint4 qv = *(const uint4*)(q8 + 128 * k + 32 * j + 16 * h + z);
        const uint32_t* qs = w + 4 + 8 * k + 4 * h;
        const uint32_t m = 0x03030303u << (2 * j);
        int32_t s = 0;
        if (j < 3) {
          s = dot4(qs[0] & m, qv.x, s);
          s = dot4(qs[1] & m, qv.y, s);
          s = dot4(qs[2] & m, qv.z, s);
          s = dot4(qs[3] & m, qv.w, s);
        } else {
          s = dot4((qs[0] >> 6) & 0x03030303u, qv.x, s);
          s = dot4((qs[1] >> 6) & 0x03030303u, qv.y, s);
          s = dot4((qs[2] >> 6) & 0x03030303u, qv.z, s);
          s = dot4((qs[3] >> 6) & 0x03030303u, qv.w, s);
        }
        acc[j] += (int32_t)sc * s;
      }
    }
  }
  const int32_t isum = acc[0] + (acc[1] >> 2) + (acc[2] >> 4) + acc[3];
  const float dall = yd * f16_to_f32_ftz((uint16_t)(w[20] & 0xFFFF));
  const float dmin = yd * f16_to_f32_ftz((uint16_t)(w[20] >> 16));
  return dall * (float)isum - dmin * (float)summs;
}

__device__ __forceinline__ int8_t sat_i8_trunc(float v) {
  if (v != v) return 0;
  if (v >= 127.0f) return 127;
  if (v <= -128.0f) return -128;
  return (int8_t)(int)v;
}

// Stage the Q8_K blocks of one activation row into LDS: qs at kQ8Stride,
// scales and (optionally) bsums beside them.  The words are fetched in
// batches of 8 per thread with every load of a batch issued before the first
// is used: coherent loads travel to memory, and one round trip per batch
// instead of one per word is what keeps the staging short.
template <bool kCoh>
__device__ __forceinline__ void stage_q8k(const uint8_t* src, int nb, uint8_t* s_q8, float* s_yd, int16_t* s_bsums) {
  const int nq = nb * 64, ny = nb, total = nq + ny + (s_bsums ? nb * 8 : 0);
  auto word = [&](int i) -> const uint32_t* {
    if (i < nq) return (const uint32_t*)(src + (size_t)(i >> 6) * Q8K_BYTES + 4 + 4 * (i & 63));
    if (i < nq + ny) return (const uint32_t*)(src + (size_t)(i - nq) * Q8K_BYTES);
    const int j = i - nq - ny;
    return (const uint32_t*)(src + (size_t)(j >> 3) * Q8K_BYTES + 260 + 4 * (j & 7));
  };
  for (int base = 0; base < total; base += 8 * (int)blockDim.x) {
    uint32_t v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = ldc<kCoh>(word(min(base + k * (int)blockDim.x + (int)threadIdx.x, total - 1)));
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int i = base + k * (int)blockDim.x + (int)threadIdx.x;
      if (i >= total) continue;
      if (i < nq) *(uint32_t*)(s_q8 + (i >> 6) * kQ8Stride + 4 * (i & 63)) = v[k];
      else if (i < nq + ny) ((uint32_t*)s_yd)[i - nq] = v[k];
      else ((uint32_t*)s_bsums)[i - nq - ny] = v[k];
    }
  }
}

__device__ __forceinline__ int align_up(int v, int a) { return (v + a - 1) / a * a; }



}  // namespace

// ===========================================================================
// Roles.  A role is one reference kernel's work for one workgroup, written
// against threadIdx.x / blockDim.x and a local block index; the kernels at the
// end of this section place several roles in one grid (fused launches) or
// run one role alone (per-kernel entry points).
// ===========================================================================
namespace {

// Lane-group butterfly sum.  For the group's first lane this is the
// reference's halving tree (xor 4,2,1 == shuffle_down 4,2,1 for lane 0;
// moe.rs:35-41, matmul.rs:10-17).  All lanes of the wave must call it.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Partial of the reference's lane-strided row sum: lane l of a W-lane group
// adds v[l], v[l+W], ... in order.
template <int W>
__device__ __forceinline__ float lane_partial(const float* v, int nb, int l) {
  float a = 0.0f;
  for (int b = l; b < nb; b += W) a += v[b];
  return a;
}

__device__ __forceinline__ uint32_t ord_f32(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---------------------------------------------------------------------------
// Router logits: matmul.rs:57-105 (matmul_f16).  256 threads per expert row
// and up to 8 tokens; thread tx sums elements tx, tx+256, ... in order and the
// LDS halving tree 128..1 combines the 256 partials, per token.
// ---------------------------------------------------------------------------
// LDS: 8 x 256 floats (the host's router_lds).  Thread tx loads its reference-order elements of
// the f16 row (each wave-wide load is one 128-byte line) and of the first
// token's x together, so the row's HBM latency and x's cache latency overlap.
template <bool kCoh>
__device__ __forceinline__ void role_router_logits(const RouterLogitsArgs& a, int bx, uint8_t* smem) {
  const int row = bx % a.E, t0 = (bx / a.E) * 8, tx = threadIdx.x;
  const int nt = min(8, a.T - t0);
  // f16 input denormals flushed for this wave (it runs no other role): the
  // hardware widening of the weights is then the reference's conversion, a
  // signed zero for every subnormal (the value only enters a multiply, so a
  // quieted signalling NaN gives the same product bits)
  __builtin_amdgcn_s_setreg(kHwregModeF16F64Denorm, 0);
  auto widen = [](uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); };
  const int d = a.d;  // d % 256 == 0 checked on the host
  const int nb = d >> 8;
  float (*part)[256] = (float (*)[256])smem;
  const uint16_t* wr = a.w + (size_t)row * d + tx;
  if (nb > 32) {
    // wide rows (the HC mix, d = 4 x 4096): the same per-thread order, one
    // element at a time
    for (int t = 0; t < nt; t++) {
      const float* xr = a.x + (size_t)(t0 + t) * d + tx;
      float acc = 0.0f;
      for (int j = 0; j < nb; j++) acc = acc + widen(wr[256 * j]) * xr[256 * j];
      part[t][tx] = acc;
    }
  } else {
  uint32_t wh[32];
  float xv[32];
  {
    const float* xr = a.x + (size_t)t0 * d + tx;
#pragma unroll
    for (int j = 0; j < 32; j++) {
      wh[j] = wr[256 * min(j, nb - 1)];
      xv[j] = xr[256 * min(j, nb - 1)];
    }
  }
  float w[32];
#pragma unroll
  for (int j = 0; j < 32; j++) w[j] = widen((uint16_t)wh[j]);
  for (int t = 0; t < nt; t++) {
    if (t > 0) {
      const float* xr = a.x + (size_t)(t0 + t) * d + tx;
#pragma unroll
      for (int j = 0; j < 32; j++) xv[j] = xr[256 * min(j, nb - 1)];
    }
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) {
      const float pr = w[j] * xv[j];
      acc = (j < nb) ? acc + pr : acc;
    }
    part[t][tx] = acc;
  }
  }
  __syncthreads();
  // halving tree: levels 128 and 64 cross waves (LDS), levels 32..1 inside
  // wave 0 (shuffle down: lane l adds lane l + s, the same pairs in the same order)
  for (int s2 = 128; s2 >= 64; s2 >>= 1) {
    if (tx < s2)
      for (int t = 0; t < nt; t++) part[t][tx] += part[t][tx + s2];
    __syncthreads();
  }
  if (tx < 64) {
    for (int t = 0; t < nt; t++) {
      float v = part[t][tx];
#pragma unroll
      for (int s2 = 32; s2 > 0; s2 >>= 1) v += __shfl_down(v, s2, 64);
      if (tx == 0) stc<kCoh>(a.out + (size_t)(t0 + t) * a.E + row, v);
    }
  }
}

// ---------------------------------------------------------------------------
// Q8_K activation quantization: quantize.rs:309-417, one 256-thread
// workgroup per 256-element block.  The signed-amax halving tree with strict
// '>' is the reference's.
// ---------------------------------------------------------------------------
// LDS: 2 x 256 floats + 256 bytes.  kCin / kCout: coherent input / output.
template <bool kCin, bool kCout>
__device__ __forceinline__ void role_q8k(const Q8KArgs& a, int bx, uint8_t* smem) {
  float* s_abs = (float*)smem;
  float* s_val = s_abs + 256;
  int8_t* s_q = (int8_t*)(s_val + 256);
  const int nb = a.in_dim >> 8;
  const int b = bx % nb, row = bx / nb, tid = threadIdx.x;
  const float v = ldc<kCin>(a.x + (size_t)row * a.in_dim + (size_t)b * 256 + tid);
  s_abs[tid] = v < 0.0f ? -v : v;
  s_val[tid] = v;
  __syncthreads();
  for (int s2 = 128; s2 > 0; s2 >>= 1) {
    if (tid < s2 && s_abs[tid + s2] > s_abs[tid]) {
      s_abs[tid] = s_abs[tid + s2];
      s_val[tid] = s_val[tid + s2];
    }
    __syncthreads();
  }
  uint8_t* yb = a.out + ((size_t)row * nb + b) * Q8K_BYTES;
  const float amax = s_abs[0];
  const float iscale = amax == 0.0f ? 0.0f : -127.0f / s_val[0];
  int8_t q = 0;
  if (amax != 0.0f) {
    const float raw = iscale * v;
    q = sat_i8_trunc(raw >= 0.0f ? raw + 0.5f : raw - 0.5f);
  }
  s_q[tid] = q;
  if (a.out_h) a.out_h[(size_t)row * a.in_dim + (size_t)b * 256 + tid] = __builtin_bit_cast(uint16_t, (_Float16)q);
  if (a.out_8) a.out_8[(size_t)row * a.in_dim + (size_t)b * 256 + tid] = q;
  __syncthreads();
  if (a.bsum_h && tid < 16) {
    int32_t s = 0;
    for (int k = 0; k < 16; k++) s += s_q[tid * 16 + k];
    a.bsum_h[(size_t)row * (a.in_dim >> 4) + (size_t)b * 16 + tid] = __builtin_bit_cast(uint16_t, (_Float16)s);
  }
  // dword stores: qs (64), bsums (8 words of two int16), d
  if (tid < 64) {
    stc<kCout>((uint32_t*)(yb + 4) + tid, ((const uint32_t*)s_q)[tid]);
  } else if (tid < 72) {
    const int j = (tid - 64) * 2;
    int32_t s0 = 0, s1 = 0;
    for (int k = 0; k < 16; k++) { s0 += s_q[j * 16 + k]; s1 += s_q[(j + 1) * 16 + k]; }
    stc<kCout>((uint32_t*)(yb + 260) + (tid - 64), (uint32_t)(uint16_t)(int16_t)s0 | ((uint32_t)(uint16_t)(int16_t)s1 << 16));
  } else if (tid == 72) {
    stc<kCout>((float*)yb, amax == 0.0f ? 0.0f : 1.0f / iscale);
  }
}

// ---------------------------------------------------------------------------
// Q8_0 activation quantization: quantize.rs:147-225.  Eight 32-element blocks
// per 256-thread workgroup.
// ---------------------------------------------------------------------------
// LDS: 8 x 32 floats + 256 bytes.  kCin / kCout: coherent input / output.
template <bool kCin, bool kCout>
__device__ __forceinline__ void role_q80(const Q80Args& a, int bx, uint8_t* smem) {
  float (*s_a)[32] = (float (*)[32])smem;
  int8_t* s_q = (int8_t*)(smem + 8 * 32 * 4);
  const int nb = (a.in_dim + 31) / 32, nwg = (nb + 7) / 8;
  const int g = threadIdx.x >> 5, tid = threadIdx.x & 31;
  const int b = (bx % nwg) * 8 + g, row = bx / nwg;
  const bool live = b < nb;
  const int i0 = b * 32;
  const int bn = live ? min(32, a.in_dim - i0) : 0;
  const float v = tid < bn ? ldc<kCin>(a.x + (size_t)row * a.in_dim + i0 + tid) : 0.0f;
  s_a[g][tid] = v < 0.0f ? -v : v;
  __syncthreads();
  for (int s2 = 16; s2 > 0; s2 >>= 1) {
    if (tid < s2 && s_a[g][tid + s2] > s_a[g][tid]) s_a[g][tid] = s_a[g][tid + s2];
    __syncthreads();
  }
  const float d = s_a[g][0] / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  int8_t q = 0;
  if (tid < bn) {
    const float raw = v * id;
    q = sat_i8_trunc(raw >= 0.0f ? raw + 0.5f : raw - 0.5f);
  }
  s_q[threadIdx.x] = q;
  if (a.out_h && live) a.out_h[(size_t)row * nb * 32 + i0 + tid] = __builtin_bit_cast(uint16_t, (_Float16)q);
  __syncthreads();
  // dword stores: 8 per block, then the scales
  const int t = threadIdx.x;
  if (t < 64) {
    const int gb = t >> 3, wd = t & 7, bb = (bx % nwg) * 8 + gb;
    if (bb < nb) stc<kCout>((uint32_t*)(a.xq + ((size_t)row * nb + bb) * 32) + wd, ((const uint32_t*)s_q)[t]);
  } else if (t < 72) {
    const int gb = t - 64, bb = (bx % nwg) * 8 + gb;
    if (bb < nb) stc<kCout>(a.xscale + (size_t)row * nb + bb, s_a[gb][0] / 127.0f);
  }
}

// ---------------------------------------------------------------------------
// The same two quantizations for batches, without LDS or barriers.
// Q8_K: one wave per 256-element block, four blocks per 256-thread
// workgroup; lane l holds elements 4l .. 4l+3.  The signed-amax halving tree
// pairs element i with i + s for s = 128 .. 1 exactly as role_q8k does: for
// s >= 4 that is lane l with lane l + s/4 (shuffle down), s = 2 and 1 are
// inside lane 0; ties keep the lower element (strict '>').  Block sums of 16
// elements are integer sums over four lanes (exact in any order).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float amax_pick(float cur, float other) {
  const float ac = cur < 0.0f ? -cur : cur, ao = other < 0.0f ? -other : other;
  return ao > ac ? other : cur;
}
__device__ __forceinline__ int8_t quant_i8(float raw) { return sat_i8_trunc(raw >= 0.0f ? raw + 0.5f : raw - 0.5f); }

// One Q8_K block `gb` (row gb / nb, block gb % nb) by the calling wave.
// kCin: the rows were stored by other workgroups of this launch (coherent
// loads).
template <bool kCin>
__device__ __forceinline__ void q8k_block_wave(const Q8KArgs& a, int gb) {
  const int nb = a.in_dim >> 8, lane = threadIdx.x & 63;
  const int b = gb % nb, row = gb / nb;
  const size_t off = (size_t)row * a.in_dim + (size_t)b * 256 + 4 * lane;
  float4 v;
  if constexpr (kCin) {
    v.x = ldc<true>(a.x + off);
    v.y = ldc<true>(a.x + off + 1);
    v.z = ldc<true>(a.x + off + 2);
    v.w = ldc<true>(a.x + off + 3);
  } else {
    v = *(const float4*)(a.x + off);
  }
  float c0 = v.x, c1 = v.y, c2 = v.z, c3 = v.w;
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    c0 = amax_pick(c0, __shfl_down(c0, s, 64));
    c1 = amax_pick(c1, __shfl_down(c1, s, 64));
    c2 = amax_pick(c2, __shfl_down(c2, s, 64));
    c3 = amax_pick(c3, __shfl_down(c3, s, 64));
  }
  c0 = amax_pick(c0, c2);
  c1 = amax_pick(c1, c3);
  c0 = amax_pick(c0, c1);
  const float best = __shfl(c0, 0, 64);
  const float amax = best < 0.0f ? -best : best;
  const float iscale = amax == 0.0f ? 0.0f : -127.0f / best;
  int8_t q[4] = {0, 0, 0, 0};
  if (amax != 0.0f) {
    q[0] = quant_i8(iscale * v.x);
    q[1] = quant_i8(iscale * v.y);
    q[2] = quant_i8(iscale * v.z);
    q[3] = quant_i8(iscale * v.w);
  }
  uint8_t* yb = a.out + ((size_t)row * nb + b) * Q8K_BYTES;
  const uint32_t packed = (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) | ((uint32_t)(uint8_t)q[2] << 16) |
                          ((uint32_t)(uint8_t)q[3] << 24);
  ((uint32_t*)(yb + 4))[lane] = packed;
  if (a.out_h) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 hv = {(_Float16)q[0], (_Float16)q[1], (_Float16)q[2], (_Float16)q[3]};
    *(h4*)(a.out_h + off) = hv;
  }
  if (a.out_8) *(uint32_t*)(a.out_8 + off) = packed;
  int32_t s = (int32_t)q[0] + q[1] + q[2] + q[3];
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  if (a.bsum_h && (lane & 3) == 0)  // the 16-element group lane / 4 (|s| <= 2032: exact in f16)
    a.bsum_h[(size_t)row * (a.in_dim >> 4) + (size_t)b * 16 + (lane >> 2)] = __builtin_bit_cast(uint16_t, (_Float16)s);
  const int32_t s_next = __shfl_down(s, 4, 64);  // the next 16-element group
  if ((lane & 7) == 0)
    ((uint32_t*)(yb + 260))[lane >> 3] = (uint32_t)(uint16_t)(int16_t)s | ((uint32_t)(uint16_t)(int16_t)s_next << 16);
  if (lane == 0) *(float*)yb = amax == 0.0f ? 0.0f : 1.0f / iscale;
}


__device__ __forceinline__ void role_q8k_waves(const Q8KArgs& a, int bx) {
  const int gb = bx * 4 + (int)(threadIdx.x >> 6);
  if (gb < (a.in_dim >> 8) * a.rows) q8k_block_wave<false>(a, gb);
}

// Q8_0: eight lanes per 32-element block (lane holds four elements), 32
// blocks per 256-thread workgroup; the abs-max tree pairs element i with
// i + s for s = 16 .. 1 as role_q80 does (s >= 4 across lanes, 2 and 1 in the
// lane).  Needs in_dim % 32 == 0.
// Blocks gb0 + (lane >> 3) (eight per wave) by the calling wave; kCin as
// for q8k_block_wave.
template <bool kCin>
__device__ __forceinline__ void q80_blocks_wave(const Q80Args& a, int gb0) {
  const int nb = a.in_dim >> 5, lane8 = threadIdx.x & 7;
  const int gb = gb0 + (int)((threadIdx.x & 63) >> 3);
  const bool live = gb < nb * a.rows;
  const int gbc = live ? gb : 0;  // dead lanes take part in the shuffles only
  const int b = gbc % nb, row = gbc / nb;
  const size_t off = (size_t)row * a.in_dim + (size_t)b * 32 + 4 * lane8;
  float4 v;
  if constexpr (kCin) {
    v.x = ldc<true>(a.x + off);
    v.y = ldc<true>(a.x + off + 1);
    v.z = ldc<true>(a.x + off + 2);
    v.w = ldc<true>(a.x + off + 3);
  } else {
    v = *(const float4*)(a.x + off);
  }
  float m0 = v.x < 0.0f ? -v.x : v.x, m1 = v.y < 0.0f ? -v.y : v.y;
  float m2 = v.z < 0.0f ? -v.z : v.z, m3 = v.w < 0.0f ? -v.w : v.w;
#pragma unroll
  for (int s = 4; s >= 1; s >>= 1) {
    float o;
    o = __shfl_down(m0, s, 8); if (o > m0) m0 = o;
    o = __shfl_down(m1, s, 8); if (o > m1) m1 = o;
    o = __shfl_down(m2, s, 8); if (o > m2) m2 = o;
    o = __shfl_down(m3, s, 8); if (o > m3) m3 = o;
  }
  if (m2 > m0) m0 = m2;
  if (m3 > m1) m1 = m3;
  if (m1 > m0) m0 = m1;
  const float amax = __shfl(m0, 0, 8);
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  const int8_t q0 = quant_i8(v.x * id), q1 = quant_i8(v.y * id), q2 = quant_i8(v.z * id), q3 = quant_i8(v.w * id);
  if (!live) return;
  ((uint32_t*)(a.xq + (size_t)row * nb * 32 + (size_t)b * 32))[lane8] =
      (uint32_t)(uint8_t)q0 | ((uint32_t)(uint8_t)q1 << 8) | ((uint32_t)(uint8_t)q2 << 16) | ((uint32_t)(uint8_t)q3 << 24);
  if (a.out_h) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 hv = {(_Float16)q0, (_Float16)q1, (_Float16)q2, (_Float16)q3};
    *(h4*)(a.out_h + off) = hv;
  }
  if (lane8 == 0) a.xscale[(size_t)row * nb + b] = amax / 127.0f;
}


__device__ __forceinline__ void role_q80_waves(const Q80Args& a, int bx) {
  q80_blocks_wave<false>(a, bx * 32 + 8 * (int)(threadIdx.x >> 6));
}

// ---------------------------------------------------------------------------
// IQ2_XXS gate + up + SwiGLU for one (row tile, pair) (moe.rs:622-715).
// Work item = one 132-byte pair of blocks of one row of gate or up; items are
// loaded before the LDS staging so their HBM latency overlaps it.  Row sums
// use 8 lanes per row in reference order; the up row's lanes sit 8 above the
// gate row's, so one shuffle brings u next to g.
// LDS: tables | yd[nb] | q8[nb][272] | vals[2][R][nb]
// ---------------------------------------------------------------------------
// Roles take a `wait` hook, called by all threads after the first weight
// loads are issued and before any activation is read; returning false skips
// the role (a dependency wait was abandoned).
struct NoWait {
  __device__ bool operator()() const { return true; }
};

__device__ __forceinline__ size_t gate_up_lds(int nb, int R) {
  return sizeof(Iq2Tables) + (size_t)align_up(nb, 4) * 4 + (size_t)nb * kQ8Stride + (size_t)2 * R * nb * 4;
}

// One work item of a gate/up tile: a 132-byte block pair of one row of the
// gate (mat 0) or up (mat 1) matrix.
struct GuItem {
  int mat, rr, m;
  bool have;
};
__device__ __forceinline__ GuItem gu_item(const GateUpArgs& a, int row0, int it) {
  const int nbp = a.d >> 9, per_mat = a.rows_per_wg * nbp;
  GuItem g;
  g.mat = it >= per_mat;
  const int rem = it - g.mat * per_mat;
  g.rr = rem / nbp;
  g.m = rem - g.rr * nbp;
  g.have = it < 2 * per_mat && row0 + g.rr < a.I;
  return g;
}
__device__ __forceinline__ void gu_load(const GateUpArgs& a, int e, int row0, const GuItem& g, uint32_t* wv) {
  if (!g.have) return;
  const size_t row_bytes = (size_t)(a.d >> 8) * IQ2XXS_BYTES;
  const uint8_t* src = (g.mat ? a.up : a.gate) + (size_t)e * a.I * row_bytes + (size_t)(row0 + g.rr) * row_bytes +
                       (size_t)g.m * 132;
#pragma unroll
  for (int q = 0; q < 8; q++) {
    const uint4 v4 = *(const uint4*)(src + 16 * q);
    wv[4 * q] = v4.x; wv[4 * q + 1] = v4.y; wv[4 * q + 2] = v4.z; wv[4 * q + 3] = v4.w;
  }
  wv[32] = *(const uint32_t*)(src + 128);
}
// LDS views of a gate/up role: tables | yd[nb] | q8[nb][272] | vals[2][R][nb]
struct GuLds {
  Iq2Tables* tab;
  float* yd;
  uint8_t* q8;
  float* vals;
};
__device__ __forceinline__ GuLds gu_lds(const GateUpArgs& a, uint8_t* smem) {
  const int nb = a.d >> 8;
  GuLds l;
  l.tab = (Iq2Tables*)smem;
  l.yd = (float*)(smem + sizeof(Iq2Tables));
  l.q8 = (uint8_t*)(l.yd + align_up(nb, 4));
  l.vals = (float*)(l.q8 + nb * kQ8Stride);
  return l;
}
__device__ __forceinline__ void gu_compute(const GateUpArgs& a, const GuItem& g, const uint32_t* wv, const GuLds& l) {
  if (!g.have) return;
  const int nb = a.d >> 8, b0 = 2 * g.m;
  const float v0 = iq2_block_dot<false>(wv, l.q8 + b0 * kQ8Stride, l.yd[b0], l.tab);
  const float v1 = iq2_block_dot<true>(wv, l.q8 + (b0 + 1) * kQ8Stride, l.yd[b0 + 1], l.tab);
  float* dst = l.vals + (g.mat * a.rows_per_wg + g.rr) * nb + b0;
  dst[0] = v0;
  dst[1] = v1;
}
// Row sums (group g = 2*rr + mat of 8 lanes, reference lane order), SwiGLU
// with the clamp, times the routing weight.
template <bool kCoh>
__device__ __forceinline__ void gu_epilogue(const GateUpArgs& a, int pair, int row0, float wgt, const GuLds& l) {
  const int nb = a.d >> 8, R = a.rows_per_wg, tid = threadIdx.x, B = blockDim.x;
  for (int base = 0; base < 2 * R * 8; base += B) {
    const int t = base + tid;
    const int grp = t >> 3, ln = t & 7;
    const int r2 = grp >> 1, mt = grp & 1;
    float p = (t < 2 * R * 8) ? lane_partial<8>(l.vals + (mt * R + r2) * nb, nb, ln) : 0.0f;
    p = group_sum<8>(p);
    const float u = __shfl_down(p, 8, 64);
    const int row = row0 + r2;
    if (t < 2 * R * 8 && ln == 0 && mt == 0 && row < a.I) {
      const float g = clamp_gate(p, a.clamp), uu = clamp_up(u, a.clamp);
      const size_t off = (size_t)pair * a.I + row;
      if (a.gate_out) a.gate_out[off] = g;
      if (a.up_out) a.up_out[off] = uu;
      stc<kCoh>(a.mid_out + off, (g / (1.0f + expf_dsm(-g))) * uu * wgt);
    }
  }
}

template <bool kCoh, class Wait = NoWait>
__device__ __forceinline__ void role_gate_up(const GateUpArgs& a, int tile, int work, uint8_t* smem, Wait wait = Wait(),
                                             bool stage = true) {
  const int nb = a.d >> 8, R = a.rows_per_wg;
  const GuLds l = gu_lds(a, smem);
  const int pair = a.pair_list ? (int)a.pair_list[work] : work;
  const int tok = pair / a.k;
  int e = a.selected ? ldc<kCoh>(a.selected + pair) : 0;
  if ((unsigned)e >= (unsigned)a.E) e = 0;  // negative ids (moe.rs:299-312) and ids past E read expert 0
  const int row0 = tile * R;
  const int items = 2 * R * (nb >> 1);
  const int B = blockDim.x;

  // first item: issue its loads before anything else
  uint32_t wv[33];
  int it = threadIdx.x;
  GuItem g = gu_item(a, row0, it);
  gu_load(a, e, row0, g, wv);
  if (!wait()) return;
  if (stage) {  // false: the tables and this token's activation are already in LDS
    load_iq2_tables(l.tab);
    stage_q8k<kCoh>(a.xq + (size_t)tok * nb * Q8K_BYTES, nb, l.q8, l.yd, nullptr);
  }
  __syncthreads();
  while (it < items) {
    gu_compute(a, g, wv, l);
    it += B;
    if (it < items) {
      g = gu_item(a, row0, it);
      gu_load(a, e, row0, g, wv);
    }
  }
  __syncthreads();
  gu_epilogue<kCoh>(a, pair, row0, a.weights ? ldc<kCoh>(a.weights + pair) : 1.0f, l);
}

// ---------------------------------------------------------------------------
// Router selection: moe.rs:177-287 (router_select_parallel) generalised to E
// experts, top-k, route_scale and group-limited selection.  One 256-thread
// workgroup per token.  The reference's insertion sort keeps the k best by
// (score desc, index asc) among scores > -inf; here every expert has a 64-bit
// key (ordered score bits, then the complemented index) and places itself by
// its rank under that order.  Group score = best + second-best biased score
// in the group.  An expert ranks below k overall only if it ranks below k in
// its group, so only each group's k best (its candidates) are ranked against
// the candidates of the kept groups: 32 comparisons per expert inside an
// 8 x 32 grouping, then 32 per candidate, no sequential arg-max rounds.
// ---------------------------------------------------------------------------
// LDS: select_lds(E) bytes; 256 threads.
__device__ __forceinline__ size_t select_lds(int E) { return (size_t)E * 20 + 128 * 4 + 64 * 4 + 32 * 8; }

__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  return ((uint64_t)readlane_u32((uint32_t)(v >> 32), l) << 32) | readlane_u32((uint32_t)v, l);
}
// Score back from the high half of a rank key (inverse of ord_f32).
__device__ __forceinline__ float key_score(uint64_t k) {
  const uint32_t u = (uint32_t)(k >> 32);
  return __builtin_bit_cast(float, (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}

template <bool kCoh>
__device__ __forceinline__ void role_select(const RouterSelectArgs& a, int t, uint8_t* smem, int32_t* s_sel = nullptr,
                                            float* s_w = nullptr, bool global = true) {
  const int E = a.E, K = a.k, G = a.n_group > 1 ? a.n_group : 1, gsz = E / G, Kc = min(K, gsz);
  const int tid = threadIdx.x;
  uint64_t* l_key = (uint64_t*)smem;  // [E]
  uint64_t* l_cand = l_key + E;       // [G][Kc]: the Kc best keys of each group, by rank
  float* l_p = (float*)(l_cand + E);  // [E]
  float* l_gb = l_p + E;              // [64][2]: best and second-best score per group
  int* l_keep = (int*)(l_gb + 128);   // [64]
  int* l_sel = l_keep + 64;           // [32]
  float* l_sp = (float*)(l_sel + 32); // [32]
  // 1. probabilities and keys, one to four experts per thread
  for (int e = tid; e < E; e += 256) {
    const float pv = __builtin_sqrtf(softplus_dsm(ldc<kCoh>(a.logits + (size_t)t * E + e)));
    const float sc = a.has_bias ? pv + a.bias[e] : pv;
    l_p[e] = pv;
    l_key[e] = sc > -__builtin_inff() ? (((uint64_t)ord_f32(sc) << 32) | (0xFFFFFFFFu - (uint32_t)e)) : 0ull;
    if (a.probs) a.probs[(size_t)t * E + e] = pv;
  }
  if (tid < 128) l_gb[tid] = -__builtin_inff();
  if (tid < 32) { l_sel[tid] = -1; l_sp[tid] = 0.0f; }
  if (G > 1)
    for (int i = tid; i < G * Kc; i += 256) l_cand[i] = 0ull;
  __syncthreads();
  // 2. rank of each expert inside its group: ranks 0 and 1 give the group
  //    score, ranks below Kc are the group's candidates (with one group, the
  //    rank is the slot)
  for (int e = tid; e < E; e += 256) {
    const uint64_t k0 = l_key[e];
    if (!k0) continue;
    const int g = e / gsz, base = g * gsz;
    int r = 0;
#pragma unroll 8
    for (int j = 0; j < gsz; j++) r += l_key[base + j] > k0;
    if (G == 1) {
      if (r < K) { l_sel[r] = e; l_sp[r] = l_p[e]; }
      continue;
    }
    if (r < 2) l_gb[2 * g + r] = key_score(k0);
    if (r < Kc) l_cand[g * Kc + r] = k0;
  }
  __syncthreads();
  const int NC = G * Kc;  // candidate slots
  int NS = 1;              // threads per candidate slot (a power of two)
  while (NS * 2 * NC <= 256 && NS < 64) NS *= 2;
  if (G > 1 && G * G <= 64) {
    // 3. kept groups, all pairs at once: lane g * G + h of wave 0 compares
    //    group h's key with group g's; the ballot's G bits of group g are its rank
    auto gkey = [&](int g) -> uint64_t {
      const float gs = gsz >= 2 ? l_gb[2 * g] + l_gb[2 * g + 1] : l_gb[2 * g];
      return gs > -__builtin_inff() ? (((uint64_t)ord_f32(gs) << 32) | (0xFFFFFFFFu - (uint32_t)g)) : 0ull;
    };
    if (tid < 64) {
      const int g = tid / G, h = tid - g * G;
      const bool act = tid < G * G;
      const uint64_t kg = act ? gkey(g) : 0ull, kh = act ? gkey(h) : 0ull;
      const uint64_t m = __ballot(act && kh > kg);
      const bool keep = act && h == 0 && kg && __popcll((m >> (g * G)) & ((1ull << G) - 1)) < a.topk_group;
      const uint64_t km = __ballot(keep);  // bit g * G for a kept group g
      // the candidates of the other groups drop out
      for (int i = tid; i < NC; i += 64)
        if (!((km >> ((i / Kc) * G)) & 1)) l_cand[i] = 0ull;
    }
    __syncthreads();
    // 4. rank of each kept candidate among the kept candidates: NS threads
    //    per candidate slot, each over a share of the slots, summed by shuffles
    const int ns_log = __builtin_ctz(NS), c = tid >> ns_log, part = tid & (NS - 1);
    const int chunk = (NC + NS - 1) >> ns_log;
    int r = 0;
    uint64_t k0 = 0ull;
    if (c < NC) {
      k0 = l_cand[c];
      if (k0) {
        const int j0 = part * chunk, j1 = min(NC, j0 + chunk);
#pragma unroll 8
        for (int j = j0; j < j1; j++) r += l_cand[j] > k0;
      }
    }
    for (int o = 1; o < NS; o <<= 1) r += __shfl_xor(r, o, 64);
    if (c < NC && part == 0 && k0 && r < K) {
      const int e = (int)(0xFFFFFFFFu - (uint32_t)k0);
      l_sel[r] = e;
      l_sp[r] = l_p[e];
    }
    __syncthreads();
  } else if (G > 1) {
    // 3. the topk_group best groups by (best + second-best score, group index)
    auto gkey = [&](int g) -> uint64_t {
      const float gs = gsz >= 2 ? l_gb[2 * g] + l_gb[2 * g + 1] : l_gb[2 * g];
      return gs > -__builtin_inff() ? (((uint64_t)ord_f32(gs) << 32) | (0xFFFFFFFFu - (uint32_t)g)) : 0ull;
    };
    if (tid < G) {
      const uint64_t mine = gkey(tid);
      int r = 0;
      for (int g2 = 0; g2 < G; g2++) r += gkey(g2) > mine;
      l_keep[tid] = mine && r < a.topk_group;
    }
    __syncthreads();
    // 4. rank of each kept candidate among all kept candidates: the slot
    for (int i = tid; i < G * Kc; i += 256) {
      const uint64_t k0 = l_cand[i];
      if (!k0 || !l_keep[i / Kc]) continue;
      int r = 0;
      for (int g2 = 0; g2 < G; g2++) {
        if (!l_keep[g2]) continue;
        for (int j = 0; j < Kc; j++) r += l_cand[g2 * Kc + j] > k0;
      }
      if (r < K) {
        const int e = (int)(0xFFFFFFFFu - (uint32_t)k0);
        l_sel[r] = e;
        l_sp[r] = l_p[e];
      }
    }
    __syncthreads();
  }
  // 5. weights: probabilities over their slot-ordered sum, times route_scale
  if (tid < K) {
    float sum = 0.0f;  // empty slots hold +0
#pragma unroll 8
    for (int j = 0; j < K; j++) sum += l_sp[j];
    if (sum < 6.103515625e-5f) sum = 6.103515625e-5f;
    const int e = l_sel[tid];
    const float wgt = (e >= 0 ? l_sp[tid] : 0.0f) / (sum / a.route_scale);
    if (global) {
      stc<kCoh>(a.selected + (size_t)t * K + tid, e);
      stc<kCoh>(a.weights + (size_t)t * K + tid, wgt);
    }
    if (s_sel) { s_sel[tid] = e; s_w[tid] = wgt; }
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// IQ2_XXS gate + up + SwiGLU, row-streaming form (moe.rs:622-715), for
// workgroups of 32 rows of one pair.  Waves 0-1 take the gate rows, waves 2-3
// the up rows; four lanes share a row and lane j (0..3) streams blocks
// j, j+4, j+8, ... of it, three blocks ahead of its arithmetic.  The
// reference's eight lane-strided partials of a row are blocks = l mod 8, so
// lane j holds partials j (even steps) and j + 4 (odd steps) in registers;
// the first level of the halving tree (xor 4) is their in-lane sum and the
// levels xor 2, xor 1 are shuffles inside the four lanes.  No block value goes
// through LDS and the only barriers are the staging and the SwiGLU hand-off.
// A block is loaded as the 17 dwords that hold it: from its own start (even
// blocks, 4-byte aligned) or from 2 bytes before it (odd blocks); every byte
// read belongs to the tensor (an even block's tail is the next block's head).
// LDS: tables | yd[nb] | q8[nb][272] | rows[2][32]
// ---------------------------------------------------------------------------
__device__ __forceinline__ size_t gate_up_rows_lds(int nb) {
  return sizeof(Iq2Tables) + (size_t)align_up(nb, 4) * 4 + (size_t)nb * kQ8Stride + 2 * 32 * 4;
}

// One IQ2_XXS block from its 17 loaded dwords; `sel` re-aligns the qs words
// (v_perm selector: bytes 2..5 for an even block, 4..7 for an odd one).
__device__ __forceinline__ float iq2_blk_dot(const uint32_t* w, uint32_t sel, uint32_t dsh, const uint8_t* q8, float yd,
                                             const Iq2Tables* t) {
  int32_t bsum = 0;
  int zo = 0;
#pragma unroll
  for (int ib = 0; ib < 8; ib++) {
    // sel and zo (always 0) pass through an empty asm that depends on the
    // running sum: the sub-block's lookups stay after the previous one's
    // arithmetic, which holds the kernel to ~116 VGPRs (4 waves per SIMD)
    // instead of 254, at no instruction for sel and one add for zo
    asm volatile("" : "+v"(sel), "+v"(zo) : "v"(bsum));
    const uint32_t aux0 = __builtin_amdgcn_perm(w[2 * ib + 1], w[2 * ib], sel);
    const uint32_t aux1 = __builtin_amdgcn_perm(w[2 * ib + 2], w[2 * ib + 1], sel);
    const uint4 qa = *(const uint4*)(q8 + ib * 32 + zo);
    const uint4 qb = *(const uint4*)(q8 + ib * 32 + 16 + zo);
    int32_t pos = 0, neg = 0;
    const uint32_t qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const uint64_t gv = t->grid[(aux0 >> (8 * g)) & 0xFF];
      const uint64_t mv = t->mask[(aux1 >> (7 * g)) & 127];
      pos = dot4((uint32_t)gv, qv[2 * g], pos);
      pos = dot4((uint32_t)(gv >> 32), qv[2 * g + 1], pos);
      neg = dot4((uint32_t)(gv & mv), qv[2 * g], neg);
      neg = dot4((uint32_t)((gv & mv) >> 32), qv[2 * g + 1], neg);
    }
    const int32_t ls = (int32_t)((aux1 >> 27) | 1u);
    // bsum += sumi * ls as one v_mad_i32_i24: |sumi| <= 3 * 32 * 43 * 128 <
    // 2^23 and ls <= 31 are inside its signed 24-bit operand range, so the
    // product is the exact one (__mul24 costs four more instructions of sign
    // extension).  The asm reads only sumi and ls, never a dot4 result: the
    // compiler inserts the wait states a DOT result needs before a VALU read
    // for its own instructions only, not for operands of inline asm.
    const int32_t sumi = pos - neg - neg;
    asm("v_mad_i32_i24 %0, %1, %2, %3" : "=v"(bsum) : "v"(sumi), "v"(ls), "v"(bsum));
  }
  // the wave runs with f16 input denormals flushed (dsmoe_up_rows): the
  // hardware widening is the reference's conversion
  const float xd = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[0] >> dsh));
  return 0.125f * xd * yd * (float)bsum;
}

#define DSM_BLK_LOAD(buf, i)                                                              \
  {                                                                                       \
    const int b_ = min(j + 4 * (i), nb - 2 + (j & 1));                                    \
    const uint8_t* src_ = wrow + (size_t)b_ * IQ2XXS_BYTES - 2 * (j & 1);                 \
    _Pragma("unroll") for (int q_ = 0; q_ < 4; q_++) {                                    \
      const uint4 v4_ = *(const uint4*)(src_ + 16 * q_);                                  \
      buf[4 * q_] = v4_.x; buf[4 * q_ + 1] = v4_.y; buf[4 * q_ + 2] = v4_.z; buf[4 * q_ + 3] = v4_.w; \
    }                                                                                     \
    buf[16] = *(const uint32_t*)(src_ + 64);                                              \
  }
__shared__ Iq2Tables g_tab_rows;

// kNit = blocks per lane, ceil(nb / 4): a compile-time count keeps every load
// unconditional and the wait counts exact.
// With `rs` (fuse_sel) the workgroup runs the token's routing (moe.rs:177-287)
// itself, into LDS, while the activation words are in flight; the workgroup
// of tile 0 of the token's first pair also stores it to rs->selected /
// rs->weights for the down launch.
__shared__ int32_t g_sel_rows[32];
__shared__ float g_wgt_rows[32];

template <int kNit>
__device__ __forceinline__ void role_gate_up_rows(const GateUpArgs& a, int tile, int pair, uint8_t* smem,
                                                  const RouterSelectArgs* rs = nullptr) {
  const int nb = a.d >> 8, tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  GuLds l = gu_lds(a, smem);
  l.tab = &g_tab_rows;  // static LDS: the table addresses fold into the lookups
  float* s_rows = (float*)(l.q8 + nb * kQ8Stride);
  const int tok = pair / a.k;

  // staging loads first (cache hits), then three blocks of weights
  const uint8_t* src = a.xq + (size_t)tok * nb * Q8K_BYTES;
  const int nq = nb * 64, total = nq + nb;
  auto word = [&](int i) -> const uint32_t* {
    return i < nq ? (const uint32_t*)(src + (size_t)(i >> 6) * Q8K_BYTES + 4 + 4 * (i & 63))
                  : (const uint32_t*)(src + (size_t)(i - nq) * Q8K_BYTES);
  };
  uint32_t sv[8];
#pragma unroll
  for (int k = 0; k < 8; k++) sv[k] = *word(min(k * 256 + tid, total - 1));
  const uint64_t grow = kIq2xxsGrid[tid & 255];

  int e;
  float wgt;
  if (rs) {
    // LDS scratch of the selection: the dynamic area, written by the staging
    // only after the selection's last barrier
    role_select<false>(*rs, tok, smem, g_sel_rows, g_wgt_rows, tile == 0 && pair % a.k == 0);
    e = g_sel_rows[pair % a.k];
    wgt = g_wgt_rows[pair % a.k];
  } else {
    e = a.selected ? a.selected[pair] : 0;
    wgt = a.weights ? a.weights[pair] : 1.0f;
  }
  if ((unsigned)e >= (unsigned)a.E) e = 0;  // negative ids (moe.rs:299-312) and ids past E read expert 0
  const int row0 = tile * 32, mat = wv >> 1, rr = (wv & 1) * 16 + (lane >> 2), j = lane & 3;
  const int row = min(row0 + rr, a.I - 1);
  const size_t row_bytes = (size_t)nb * IQ2XXS_BYTES;
  const uint8_t* wrow = (mat ? a.up : a.gate) + ((size_t)e * a.I + row) * row_bytes;
  const uint32_t sel = (j & 1) ? 0x07060504u : 0x05040302u, dsh = (j & 1) ? 16u : 0u;
  uint32_t wb[3][17];
#pragma unroll
  for (int i = 0; i < 3 && i < kNit; i++) DSM_BLK_LOAD(wb[i], i)
  if (tid < 128) l.tab->mask[tid] = sign_mask64(iq2_sign_byte(tid));
  l.tab->grid[tid & 255] = grow;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int i = k * 256 + tid;
    if (i < nq) *(uint32_t*)(l.q8 + (i >> 6) * kQ8Stride + 4 * (i & 63)) = sv[k];
    else if (i < total) ((uint32_t*)l.yd)[i - nq] = sv[k];
  }
  for (int i = 2048 + tid; i < total; i += 256) {  // d > 8160 only
    if (i < nq) *(uint32_t*)(l.q8 + (i >> 6) * kQ8Stride + 4 * (i & 63)) = *word(i);
    else ((uint32_t*)l.yd)[i - nq] = *word(i);
  }
  __syncthreads();

  float p_lo = 0.0f, p_hi = 0.0f;
#pragma unroll
  for (int i = 0; i < kNit; i++) {
    const int b = j + 4 * i;
    if (b < nb) {
      const float v = iq2_blk_dot(wb[i % 3], sel, dsh, l.q8 + b * kQ8Stride, l.yd[b], l.tab);
      if (i & 1) p_hi += v; else p_lo += v;
    }
    if (i + 3 < kNit) DSM_BLK_LOAD(wb[i % 3], i + 3)
  }
  float q = p_lo + p_hi;              // halving tree, level xor 4 (in-lane)
  q += __shfl_xor(q, 2, 64);          // level xor 2
  q += __shfl_xor(q, 1, 64);          // level xor 1
  if (j == 0) s_rows[mat * 32 + rr] = q;
  __syncthreads();
  if (tid < 32 && row0 + tid < a.I) {
    const float g = clamp_gate(s_rows[tid], a.clamp), uu = clamp_up(s_rows[32 + tid], a.clamp);
    const size_t off = (size_t)pair * a.I + row0 + tid;
    if (a.gate_out) a.gate_out[off] = g;
    if (a.up_out) a.up_out[off] = uu;
    // device-coherent: a workgroup of this launch may quantize the row block
    stc<true>(a.mid_out + off, (g / (1.0f + expf_dsm(-g))) * uu * wgt);
  }
}

// ---------------------------------------------------------------------------
// Expert-major gate/up/SwiGLU (batches with few pairs per expert; the
// reference's moe_gate_up_mid_sorted_qwarp32, moe.rs:721-815, per-pair
// arithmetic of :622-715).  A workgroup takes one chunk of up to m.np pairs
// of one expert (a dsmoe_dispatch tile with block_m = m.np <= kEmPairs) and
// 32 rows of gate and of up: the weight rows stream once, in the
// row-streaming layout above (4 lanes per row, lane j takes blocks j, j+4,
// ...), and every decoded block is multiplied with the activations of the
// chunk's pairs, staged in LDS (the pair loop runs the chunk's count; a
// branch-free loop over a compiled count let the compiler hoist every
// lookup and spill).  The signs go onto the
// grid bytes before the products (exact: every signed grid byte is in
// [-43, 43]), so a pair costs two dot4 per 8 weights.  Each pair's sum keeps
// the reference's order (block classes j and j+4 in-lane, then xor 2, xor
// 1), so the bits equal the per-pair kernels'.
// LDS (all dynamic): tables | q8[m.np][nb][272] (each block's d in bytes
// 256..259 of its padding); the row sums reuse the q8 space after the
// products.
// ---------------------------------------------------------------------------

// Signed grid bytes of 8 weights: byte i is -g_i where mask byte i is 0xFF.
// 0x01010100 - g negates every byte at once (no byte of g is 0, so each
// byte borrows exactly one from the next).
__device__ __forceinline__ uint32_t signed_grid4(uint32_t g, uint32_t m) {
  const uint32_t neg = 0x01010100u - g;
  return (neg & m) | (g & ~m);
}

template <int kNit>
__device__ __forceinline__ void role_gate_up_em(const GuEmArgs& m, int tile, int e, int p0, int cnt, uint8_t* smem) {
  constexpr int NP = kEmPairs;
  const GateUpArgs& a = m.gu;
  const int nb = a.d >> 8, tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  Iq2Tables* tab = (Iq2Tables*)smem;
  uint8_t* s_q8 = smem + sizeof(Iq2Tables);  // [np][nb][272]
  float* s_rows = (float*)s_q8;              // [NP][64], after the products

  const int row0 = tile * 32, mat = wv >> 1, rr = (wv & 1) * 16 + (lane >> 2), j = lane & 3;
  const int row = min(row0 + rr, a.I - 1);
  const size_t row_bytes = (size_t)nb * IQ2XXS_BYTES;
  const uint8_t* wrow = (mat ? a.up : a.gate) + ((size_t)e * a.I + row) * row_bytes;
  const uint32_t sel = (j & 1) ? 0x07060504u : 0x05040302u, dsh = (j & 1) ? 16u : 0u;
  uint32_t wb[3][17];
#pragma unroll
  for (int i = 0; i < 3 && i < kNit; i++) DSM_BLK_LOAD(wb[i], i)
  if (tid < 128) tab->mask[tid] = sign_mask64(iq2_sign_byte(tid));
  tab->grid[tid & 255] = kIq2xxsGrid[tid & 255];
  // activations of the chunk's pairs: per pair nb * 64 qs words then nb d
  // words, eight independent loads in flight per thread before their stores
  const int per = nb * 65;
#pragma unroll
  for (int q = 0; q < NP; q++) {
    if (q < cnt) {
      const uint8_t* src = a.xq + (size_t)(m.sorted_pairs[p0 + q] / (uint32_t)a.k) * nb * Q8K_BYTES;
      uint8_t* dst = s_q8 + (size_t)q * nb * kQ8Stride;
      for (int i0 = 0; i0 < per; i0 += 8 * 256) {
        uint32_t v[8];
#pragma unroll
        for (int t = 0; t < 8; t++) {
          const int r = min(i0 + t * 256 + tid, per - 1);
          v[t] = r < nb * 64 ? *(const uint32_t*)(src + (size_t)(r >> 6) * Q8K_BYTES + 4 + 4 * (r & 63))
                             : *(const uint32_t*)(src + (size_t)(r - nb * 64) * Q8K_BYTES);
        }
#pragma unroll
        for (int t = 0; t < 8; t++) {
          const int r = i0 + t * 256 + tid;
          if (r < nb * 64) *(uint32_t*)(dst + (r >> 6) * kQ8Stride + 4 * (r & 63)) = v[t];
          else if (r < per) *(uint32_t*)(dst + (r - nb * 64) * kQ8Stride + 256) = v[t];
        }
      }
    }
  }
  __syncthreads();

  float p_lo[NP], p_hi[NP];
#pragma unroll
  for (int q = 0; q < NP; q++) { p_lo[q] = 0.0f; p_hi[q] = 0.0f; }
#pragma unroll
  for (int i = 0; i < kNit; i++) {
    const int b = j + 4 * i;
    if (b < nb) {
      const uint32_t* w = wb[i % 3];
      int32_t bsum[NP];
#pragma unroll
      for (int q = 0; q < NP; q++) bsum[q] = 0;
#pragma unroll
      for (int ib = 0; ib < 8; ib++) {
        const uint32_t aux0 = __builtin_amdgcn_perm(w[2 * ib + 1], w[2 * ib], sel);
        const uint32_t aux1 = __builtin_amdgcn_perm(w[2 * ib + 2], w[2 * ib + 1], sel);
        uint32_t sg[8];
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const uint64_t gv = tab->grid[(aux0 >> (8 * g)) & 0xFF];
          const uint64_t mv = tab->mask[(aux1 >> (7 * g)) & 127];
          sg[2 * g] = signed_grid4((uint32_t)gv, (uint32_t)mv);
          sg[2 * g + 1] = signed_grid4((uint32_t)(gv >> 32), (uint32_t)(mv >> 32));
        }
        const int32_t ls = (int32_t)((aux1 >> 27) | 1u);
#pragma unroll
        for (int q = 0; q < NP; q++) {
          if (q >= cnt) break;
          const uint8_t* q8 = s_q8 + ((size_t)q * nb + b) * kQ8Stride + ib * 32;
          const uint4 qa = *(const uint4*)q8, qb = *(const uint4*)(q8 + 16);
          int32_t sumi = dot4(sg[0], qa.x, 0);
          sumi = dot4(sg[1], qa.y, sumi);
          sumi = dot4(sg[2], qa.z, sumi);
          sumi = dot4(sg[3], qa.w, sumi);
          sumi = dot4(sg[4], qb.x, sumi);
          sumi = dot4(sg[5], qb.y, sumi);
          sumi = dot4(sg[6], qb.z, sumi);
          sumi = dot4(sg[7], qb.w, sumi);
          bsum[q] += __mul24(sumi, ls);  // |sumi| < 2^18, ls <= 31
        }
      }
      const float xd = f16_to_f32_ftz((uint16_t)(w[0] >> dsh));
#pragma unroll
      for (int q = 0; q < NP; q++) {
        if (q >= cnt) break;
        const float yd = *(const float*)(s_q8 + ((size_t)q * nb + b) * kQ8Stride + 256);
        const float v = 0.125f * xd * yd * (float)bsum[q];
        if (i & 1) p_hi[q] += v; else p_lo[q] += v;
      }
    }
    if (i + 3 < kNit) DSM_BLK_LOAD(wb[i % 3], i + 3)
  }
  __syncthreads();  // every wave is done with the staged activations
#pragma unroll
  for (int q = 0; q < NP; q++) {
    if (q >= cnt) break;
    float v = p_lo[q] + p_hi[q];   // halving tree, level xor 4 (in-lane)
    v += __shfl_xor(v, 2, 64);     // level xor 2
    v += __shfl_xor(v, 1, 64);     // level xor 1
    if (j == 0) s_rows[q * 64 + mat * 32 + rr] = v;
  }
  __syncthreads();
  for (int i = tid; i < cnt * 32; i += 256) {
    const int q = i >> 5, r = i & 31;
    if (row0 + r >= a.I) continue;
    const uint32_t pair = m.sorted_pairs[p0 + q];
    const float g = clamp_gate(s_rows[q * 64 + r], a.clamp), uu = clamp_up(s_rows[q * 64 + 32 + r], a.clamp);
    const float wgt = a.weights ? a.weights[pair] : 1.0f;
    a.mid_out[(size_t)pair * a.I + row0 + r] = (g / (1.0f + expf_dsm(-g))) * uu * wgt;
  }
}
#undef DSM_BLK_LOAD



// ---------------------------------------------------------------------------
// Q2_K down projection + slot-ordered sum for one (row tile, token)
// (moe.rs:821-866, :922-970, :983-1005).  Work item = one 84-byte block.
// LDS: yd[K*nb] | bsums[K*nb][16] | q8[K*nb][272] | vals[K][R][nb] | acc[K][R]
// ---------------------------------------------------------------------------
template <bool kCoh, class Wait = NoWait>
__device__ __forceinline__ void role_down(const DownArgs& a, int tile, int tok, uint8_t* smem, Wait wait = Wait(), bool stage = true) {
  const int nb = a.I >> 8, R = a.rows_per_wg, K = a.k;
  float* s_yd = (float*)smem;
  int16_t* s_bs = (int16_t*)(s_yd + align_up(K * nb, 4));
  uint8_t* s_q8 = (uint8_t*)(s_bs + K * nb * 16);
  float* s_vals = (float*)(s_q8 + K * nb * kQ8Stride);
  float* s_acc = s_vals + K * R * nb;

  const int row0 = tile * R;
  const size_t row_bytes = (size_t)nb * Q2K_BYTES;
  const size_t exp_bytes = (size_t)a.d * row_bytes;
  const int per_slot = R * nb;
  const int items = K * per_slot;
  const int tid = threadIdx.x, B = blockDim.x;

  uint32_t wv[21];
  int it = tid, s = 0, rr = 0, b = 0;
  bool have = false;
  auto load_item = [&](int it_) {
    s = it_ / per_slot;
    const int rem = it_ - s * per_slot;
    rr = rem / nb;
    b = rem - rr * nb;
    have = row0 + rr < a.d;
    if (!have) return;
    int e = a.selected ? ldc<kCoh>(a.selected + tok * K + s) : 0;
    if ((unsigned)e >= (unsigned)a.E) e = 0;  // negative ids (moe.rs:299-312) and ids past E read expert 0
    const uint8_t* src = a.down + (size_t)e * exp_bytes + (size_t)(row0 + rr) * row_bytes + (size_t)b * Q2K_BYTES;
#pragma unroll
    for (int q = 0; q < 5; q++) {
      const uint4 v4 = *(const uint4*)(src + 16 * q);
      wv[4 * q] = v4.x; wv[4 * q + 1] = v4.y; wv[4 * q + 2] = v4.z; wv[4 * q + 3] = v4.w;
    }
    wv[20] = *(const uint32_t*)(src + 80);
  };
  if (it < items) load_item(it);
  if (!wait()) return;

  if (stage) stage_q8k<kCoh>(a.midq + (size_t)tok * K * nb * Q8K_BYTES, K * nb, s_q8, s_yd, s_bs);
  __syncthreads();

  while (it < items) {
    if (have) {
      const int qb = s * nb + b;
      s_vals[(s * R + rr) * nb + b] = q2k_block_dot(wv, s_q8 + qb * kQ8Stride, s_bs + qb * 16, s_yd[qb]);
    }
    it += B;
    if (it < items) load_item(it);
  }
  __syncthreads();

  for (int base = 0; base < K * R * 8; base += B) {
    const int t = base + tid;
    const int grp = t >> 3, l = t & 7;
    const int ss = grp / R, r2 = grp - ss * R;
    float p = (t < K * R * 8) ? lane_partial<8>(s_vals + (ss * R + r2) * nb, nb, l) : 0.0f;
    p = group_sum<8>(p);
    if (t < K * R * 8 && l == 0) {
      s_acc[ss * R + r2] = p;
      if (a.down_out && row0 + r2 < a.d) a.down_out[((size_t)tok * K + ss) * a.d + row0 + r2] = p;
    }
  }
  __syncthreads();
  if (a.out)
    for (int r2 = tid; r2 < R; r2 += B) {
      if (row0 + r2 >= a.d) continue;
      float total = 0.0f;
      for (int ss = 0; ss < K; ss++) total += s_acc[ss * R + r2];
      a.out[(size_t)tok * a.d + row0 + r2] = total;
    }
}

// Q2_K down projection + slot-ordered sum, row-streaming form (k <= 8):
// lane l of a wave takes slot l / 8 and blocks l % 8, l % 8 + 8, ... (the
// reference's partial l % 8) of kRpw rows (rows w, w + 4, ... of the tile),
// all loaded up front; the 8-lane butterfly gives the slot sums and lane 0
// adds them in slot order.  No block value goes through LDS.
// LDS: yd[K*nb] | bsums[K*nb][16] | q8[K*nb][272]
template <int kNit, int kRpw>
__device__ __forceinline__ void role_down_rows(const DownArgs& a, int tile, int tok, uint8_t* smem) {
  const int nb = a.I >> 8, K = a.k, tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  float* s_yd = (float*)smem;
  int16_t* s_bs = (int16_t*)(s_yd + align_up(K * nb, 4));
  uint8_t* s_q8 = (uint8_t*)(s_bs + K * nb * 16);
  const int slot = lane >> 3, j = lane & 7, sl = min(slot, K - 1);
  int e = a.selected ? a.selected[tok * K + sl] : 0;
  if ((unsigned)e >= (unsigned)a.E) e = 0;  // negative ids (moe.rs:299-312) and ids past E read expert 0
  const size_t row_bytes = (size_t)nb * Q2K_BYTES;
  const int row0 = tile * 4 * kRpw;
  // the activation words are loaded first (cache hits) so that the LDS
  // stores and the barrier wait for them alone, not for the weights
  const uint8_t* xsrc = a.midq + (size_t)tok * K * nb * Q8K_BYTES;
  const int nqb = K * nb, nq = nqb * 64, ny = nqb, total = nq + ny + nqb * 8;
  auto word = [&](int i) -> const uint32_t* {
    if (i < nq) return (const uint32_t*)(xsrc + (size_t)(i >> 6) * Q8K_BYTES + 4 + 4 * (i & 63));
    if (i < nq + ny) return (const uint32_t*)(xsrc + (size_t)(i - nq) * Q8K_BYTES);
    const int jj = i - nq - ny;
    return (const uint32_t*)(xsrc + (size_t)(jj >> 3) * Q8K_BYTES + 260 + 4 * (jj & 7));
  };
  constexpr int kSv = 19;  // covers k * nb <= 64 blocks (73 words each) with 256 threads
  uint32_t sv[kSv];
#pragma unroll
  for (int c = 0; c < kSv; c++) sv[c] = *word(min(c * 256 + tid, total - 1));
  uint32_t wb[kRpw][kNit][21];
#pragma unroll
  for (int q = 0; q < kRpw; q++) {
    const int row = min(row0 + wv + 4 * q, a.d - 1);
    const uint8_t* wrow = a.down + ((size_t)e * a.d + row) * row_bytes;
#pragma unroll
    for (int i = 0; i < kNit; i++) {
      const uint8_t* src = wrow + (size_t)min(j + 8 * i, nb - 1) * Q2K_BYTES;
#pragma unroll
      for (int c = 0; c < 5; c++) {
        const uint4 v4 = *(const uint4*)(src + 16 * c);
        wb[q][i][4 * c] = v4.x; wb[q][i][4 * c + 1] = v4.y; wb[q][i][4 * c + 2] = v4.z; wb[q][i][4 * c + 3] = v4.w;
      }
      wb[q][i][20] = *(const uint32_t*)(src + 80);
    }
  }
#pragma unroll
  for (int c = 0; c < kSv; c++) {
    const int i = c * 256 + tid;
    if (i < nq) *(uint32_t*)(s_q8 + (i >> 6) * kQ8Stride + 4 * (i & 63)) = sv[c];
    else if (i < nq + ny) ((uint32_t*)s_yd)[i - nq] = sv[c];
    else if (i < total) ((uint32_t*)s_bs)[i - nq - ny] = sv[c];
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kRpw; q++) {
    float p = 0.0f;  // the reference's lane-strided partial j of this slot's row
#pragma unroll
    for (int i = 0; i < kNit; i++) {
      const int b = j + 8 * i;
      if (b < nb && slot < K) {
        const int qb = sl * nb + b;
        p += q2k_block_dot(wb[q][i], s_q8 + qb * kQ8Stride, s_bs + qb * 16, s_yd[qb]);
      }
    }
    p = group_sum<8>(p);
    const int row = row0 + wv + 4 * q;
    if (a.down_out && j == 0 && slot < K && row < a.d) a.down_out[((size_t)tok * K + slot) * a.d + row] = p;
    float total = 0.0f;
    for (int ss = 0; ss < K; ss++) total += __shfl(p, 8 * ss, 64);
    if (a.out && lane == 0 && row < a.d) a.out[(size_t)tok * a.d + row] = total;
  }
}
__device__ __forceinline__ void role_down_rows_any(const DownArgs& a, int tile, int tok, uint8_t* smem) {
  role_down_rows<1, 2>(a, tile, tok, smem);  // I <= 2048, k <= 8 (checked on the host)
}

// Expert-major down projection (batches with few pairs per expert;
// moe_down_sorted_qwarp32, moe.rs:871-916): a workgroup takes one chunk of
// up to kEmPairs pairs of one expert and kDnEmRows rows of its down matrix,
// 32 rows per step (8 per wave), the next step's weights in flight during
// the current one.  Lane l of a wave takes row l/8 of the wave's eight and
// block l mod 8 of it (the reference's lane-strided partial), holds that
// block in registers and runs it against every pair of the chunk; the
// 8-lane butterfly finishes each pair's row and the value goes to
// down_out[pair][row] (the slot-ordered sum runs after, in dsmoe_moe_sum).
// I <= 2048 (one block per lane).
// LDS: the chunk's Q8_K(mid) blocks as copied, [kEmPairs][nb] slots of 304
// bytes starting at byte 12 of a slot (the 256 qs bytes 16-byte aligned).
__device__ __forceinline__ void role_down_em(const DnEmArgs& m, int tile, int chunk, uint8_t* smem) {
  const DownArgs& a = m.dn;
  const int nb = a.I >> 8, tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  if (chunk >= (int)m.tile_offsets[a.E]) return;
  const int e = (int)m.tile_experts[chunk];
  const int p0 = (int)(m.offsets[e] + m.tile_starts[chunk]);
  const int cnt = min(m.np, (int)m.offsets[e + 1] - p0);
  constexpr int kSlot = 304, kSteps = kDnEmRows / 32;
  const int rl = lane >> 3, j = lane & 7;
  const size_t row_bytes = (size_t)nb * Q2K_BYTES;
  const int row0 = tile * kDnEmRows + wv * 8 + rl;
  const uint8_t* wbase = a.down + (size_t)e * a.d * row_bytes + (size_t)min(j, nb - 1) * Q2K_BYTES;
  auto load = [&](int st, uint32_t (&w)[21]) {
    const uint8_t* src = wbase + (size_t)min(row0 + 32 * st, a.d - 1) * row_bytes;
#pragma unroll
    for (int c = 0; c < 5; c++) {
      const uint4 v4 = *(const uint4*)(src + 16 * c);
      w[4 * c] = v4.x; w[4 * c + 1] = v4.y; w[4 * c + 2] = v4.z; w[4 * c + 3] = v4.w;
    }
    w[20] = *(const uint32_t*)(src + 80);
  };
  uint32_t wa[21], wb[21];
  load(0, wa);
  // the chunk's Q8_K(mid) blocks, 73 words each, copied whole
  const int per = nb * 73;
#pragma unroll
  for (int q = 0; q < kEmPairs; q++) {
    if (q < cnt) {
      const uint32_t* src = (const uint32_t*)(a.midq + (size_t)m.sorted_pairs[p0 + q] * nb * Q8K_BYTES);
      uint8_t* dst = smem + (size_t)q * nb * kSlot + 12;
      for (int i0 = 0; i0 < per; i0 += 4 * 256) {
        uint32_t v[4];
#pragma unroll
        for (int t = 0; t < 4; t++) v[t] = src[min(i0 + t * 256 + tid, per - 1)];
#pragma unroll
        for (int t = 0; t < 4; t++) {
          const int r = i0 + t * 256 + tid;
          if (r < per) *(uint32_t*)(dst + (r / 73) * kSlot + 4 * (r % 73)) = v[t];
        }
      }
    }
  }
  __syncthreads();
  const uint8_t* slot0 = smem + (size_t)min(j, nb - 1) * kSlot + 12;
  auto run = [&](int st, const uint32_t (&w)[21]) {
    const int row = row0 + 32 * st;
#pragma unroll
    for (int q = 0; q < kEmPairs; q++) {
      if (q < cnt) {
        const uint8_t* blk = slot0 + (size_t)q * nb * kSlot;
        // the reference's lane-strided partial j of this pair's row
        float p = j < nb ? q2k_block_dot(w, blk + 4, (const int16_t*)(blk + 260), *(const float*)blk) : 0.0f;
        p = group_sum<8>(p);
        if (j == 0 && row < a.d) a.down_out[(size_t)m.sorted_pairs[p0 + q] * a.d + row] = p;
      }
    }
  };
#pragma unroll
  for (int st = 0; st < kSteps; st += 2) {
    load(min(st + 1, kSteps - 1), wb);
    run(st, wa);
    load(min(st + 2, kSteps - 1), wa);
    run(st + 1, wb);
  }
}

// ---------------------------------------------------------------------------
// Q8_0 matvec for one (row tile, token) (matmul.rs:357-458), one or two
// matrices; with two, SwiGLU (utils.rs:141-163, weight 1) on the pair.
// Work item = one 68-byte pair of Q8_0 blocks.  Row sums use 32 lanes per
// row in reference order.
// LDS: xs[nb] | xq[nb*32] | vals[nmat][R][nb]
// ---------------------------------------------------------------------------
template <bool kCoh, class Wait = NoWait>
__device__ __forceinline__ void role_q80_matvec(const Q80MatvecArgs& a, int tile, int tok, uint8_t* smem, Wait wait = Wait(),
                                bool stage = true) {
  const int nb = a.in_dim >> 5, nbp = nb >> 1, R = a.rows_per_wg;
  const int nmat = a.w1 ? 2 : 1;
  float* s_xs = (float*)smem;
  uint32_t* s_xq = (uint32_t*)(s_xs + align_up(nb, 4));
  float* s_vals = (float*)(s_xq + nb * 8);
  const int row0 = tile * R;
  const size_t row_bytes = (size_t)nb * Q8_0_BYTES;
  const int per_mat = R * nbp;
  const int items = nmat * per_mat;
  const int tid = threadIdx.x, B = blockDim.x;

  uint32_t wv[17];
  int it = tid, mat = 0, rr = 0, m = 0;
  bool have = false;
  auto load_item = [&](int it_) {
    mat = it_ >= per_mat;
    const int rem = it_ - mat * per_mat;
    rr = rem / nbp;
    m = rem - rr * nbp;
    have = row0 + rr < a.out_dim;
    if (!have) return;
    const uint8_t* src = (mat ? a.w1 : a.w0) + (size_t)(row0 + rr) * row_bytes + (size_t)m * 68;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint4 v4 = *(const uint4*)(src + 16 * q);
      wv[4 * q] = v4.x; wv[4 * q + 1] = v4.y; wv[4 * q + 2] = v4.z; wv[4 * q + 3] = v4.w;
    }
    wv[16] = *(const uint32_t*)(src + 64);
  };
  if (it < items) load_item(it);
  if (!wait()) return;

  if (stage) {  // batches of 8 words per thread, all loads of a batch in flight together
    const uint32_t* xq = (const uint32_t*)(a.xq + (size_t)tok * nb * 32);
    const uint32_t* xs = (const uint32_t*)(a.xscale + (size_t)tok * nb);
    const int total = nb * 9;
    for (int base = 0; base < total; base += 8 * B) {
      uint32_t v[8];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int i = min(base + k * B + tid, total - 1);
        v[k] = ldc<kCoh>(i < nb * 8 ? xq + i : xs + (i - nb * 8));
      }
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int i = base + k * B + tid;
        if (i < nb * 8) s_xq[i] = v[k];
        else if (i < total) ((uint32_t*)s_xs)[i - nb * 8] = v[k];
      }
    }
  }
  __syncthreads();

  while (it < items) {
    if (have) {
      const int b0 = 2 * m;
      int32_t d0 = 0, d1 = 0;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        d0 = dot4(alignbyte(wv[j + 1], wv[j], 2), s_xq[b0 * 8 + j], d0);
        d1 = dot4(wv[9 + j], s_xq[(b0 + 1) * 8 + j], d1);
      }
      const float sc0 = f16_to_f32_ftz((uint16_t)(wv[0] & 0xFFFF));
      const float sc1 = f16_to_f32_ftz((uint16_t)(wv[8] >> 16));
      float* dst = s_vals + (mat * R + rr) * nb + b0;
      dst[0] = sc0 * s_xs[b0] * (float)d0;
      dst[1] = sc1 * s_xs[b0 + 1] * (float)d1;
    }
    it += B;
    if (it < items) load_item(it);
  }
  __syncthreads();

  for (int base = 0; base < nmat * R * 32; base += B) {
    const int t = base + tid;
    const int grp = t >> 5, l = t & 31;
    const int r2 = nmat == 2 ? grp >> 1 : grp, mt = nmat == 2 ? grp & 1 : 0;
    float p = (t < nmat * R * 32) ? lane_partial<32>(s_vals + (mt * R + r2) * nb, nb, l) : 0.0f;
    p = group_sum<32>(p);
    const float u = __shfl_down(p, 32, 64);
    const int row = row0 + r2;
    if (t < nmat * R * 32 && l == 0 && mt == 0 && row < a.out_dim) {
      const size_t off = (size_t)tok * a.out_dim + row;
      if (nmat == 1) {
        a.out0[off] = p;
      } else {
        if (a.out0) a.out0[off] = p;
        if (a.out1) a.out1[off] = u;
        if (a.mid) {
          const float g = clamp_gate(p, a.clamp), uu = clamp_up(u, a.clamp);
          stc<kCoh>(a.mid + off, (g / (1.0f + expf_dsm(-g))) * uu * 1.0f);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Pieces of the Q8_0 matvec and Q2_K down roles for software-pipelined
// persistent loops (one work item per thread per unit; the next unit's
// weights are loaded while the current one is computed).
// ---------------------------------------------------------------------------
struct Q80Item {
  int mat, rr, m;
  bool have;
};
__device__ __forceinline__ Q80Item q80_item(const Q80MatvecArgs& a, int row0, int it) {
  const int nbp = a.in_dim >> 6, per_mat = a.rows_per_wg * nbp, nmat = a.w1 ? 2 : 1;
  Q80Item q;
  q.mat = it >= per_mat;
  const int rem = it - q.mat * per_mat;
  q.rr = rem / nbp;
  q.m = rem - q.rr * nbp;
  q.have = it < nmat * per_mat && row0 + q.rr < a.out_dim;
  return q;
}
// kLast: register slot of the pair's 17th dword.  A persistent loop that
// also holds another kind of unit in the same registers puts it in that
// kind's last slot, so both kinds fill the same slots (the compiler
// otherwise merges the two loads behind a computed index in scratch).
template <int kLast = 16>
__device__ __forceinline__ void q80_load(const Q80MatvecArgs& a, int row0, const Q80Item& q, uint32_t* wv) {
  if (!q.have) return;
  const size_t row_bytes = (size_t)(a.in_dim >> 5) * Q8_0_BYTES;
  const uint8_t* src = (q.mat ? a.w1 : a.w0) + (size_t)(row0 + q.rr) * row_bytes + (size_t)q.m * 68;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint4 v4 = *(const uint4*)(src + 16 * j);
    wv[4 * j] = v4.x; wv[4 * j + 1] = v4.y; wv[4 * j + 2] = v4.z; wv[4 * j + 3] = v4.w;
  }
  wv[kLast] = *(const uint32_t*)(src + 64);
}
// One (row tile, token) unit of the Q8_0 matvec from preloaded weights:
// stages the activation when `stage`, computes, and writes the rows.
template <bool kCoh, int kLast = 16>
__device__ __forceinline__ void q80_unit(const Q80MatvecArgs& a, int tile, int tok, uint8_t* smem, const uint32_t* wv,
                                         bool stage) {
  const int nb = a.in_dim >> 5, R = a.rows_per_wg, nmat = a.w1 ? 2 : 1, tid = threadIdx.x, B = blockDim.x;
  float* s_xs = (float*)smem;
  uint32_t* s_xq = (uint32_t*)(s_xs + align_up(nb, 4));
  float* s_vals = (float*)(s_xq + nb * 8);
  const int row0 = tile * R;
  if (stage) {
    const uint32_t* xq = (const uint32_t*)(a.xq + (size_t)tok * nb * 32);
    const uint32_t* xs = (const uint32_t*)(a.xscale + (size_t)tok * nb);
    const int total = nb * 9;
    for (int base = 0; base < total; base += 8 * B) {
      uint32_t v[8];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int i = min(base + k * B + tid, total - 1);
        v[k] = ldc<kCoh>(i < nb * 8 ? xq + i : xs + (i - nb * 8));
      }
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int i = base + k * B + tid;
        if (i < nb * 8) s_xq[i] = v[k];
        else if (i < total) ((uint32_t*)s_xs)[i - nb * 8] = v[k];
      }
    }
  }
  __syncthreads();
  const Q80Item q = q80_item(a, row0, tid);
  if (q.have) {
    const int b0 = 2 * q.m;
    int32_t d0 = 0, d1 = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      d0 = dot4(alignbyte(wv[j + 1], wv[j], 2), s_xq[b0 * 8 + j], d0);
      d1 = dot4(j < 7 ? wv[9 + j] : wv[kLast], s_xq[(b0 + 1) * 8 + j], d1);
    }
    const float sc0 = f16_to_f32_ftz((uint16_t)(wv[0] & 0xFFFF));
    const float sc1 = f16_to_f32_ftz((uint16_t)(wv[8] >> 16));
    float* dst = s_vals + (q.mat * R + q.rr) * nb + b0;
    dst[0] = sc0 * s_xs[b0] * (float)d0;
    dst[1] = sc1 * s_xs[b0 + 1] * (float)d1;
  }
  __syncthreads();
  for (int base = 0; base < nmat * R * 32; base += B) {
    const int t = base + tid;
    const int grp = t >> 5, l = t & 31;
    const int r2 = nmat == 2 ? grp >> 1 : grp, mt = nmat == 2 ? grp & 1 : 0;
    float p = (t < nmat * R * 32) ? lane_partial<32>(s_vals + (mt * R + r2) * nb, nb, l) : 0.0f;
    p = group_sum<32>(p);
    const float u = __shfl_down(p, 32, 64);
    const int row = row0 + r2;
    if (t < nmat * R * 32 && l == 0 && mt == 0 && row < a.out_dim) {
      const size_t off = (size_t)tok * a.out_dim + row;
      if (nmat == 1) {
        stc<kCoh>(a.out0 + off, p);
      } else {
        if (a.out0) a.out0[off] = p;
        if (a.out1) a.out1[off] = u;
        if (a.mid) {
          const float g = clamp_gate(p, a.clamp), uu = clamp_up(u, a.clamp);
          stc<kCoh>(a.mid + off, (g / (1.0f + expf_dsm(-g))) * uu * 1.0f);
        }
      }
    }
  }
}

// Q8_0 matvec (+ SwiGLU when w1 is given), row-streaming form
// (session.rs:2075-2112 with the reference's 32-lane row sums): 32 lanes per
// row, lane l streams blocks l, l+32, ... (the reference's partial l) with
// every block loaded up front, and the halving tree is the 32-lane butterfly.
// A tile is 8 rows of one matrix, or 4 rows of each of w0 (waves 0-1) and w1
// (waves 2-3).  Blocks are loaded as the 9 dwords that hold them (from 2
// bytes before an odd block), every byte inside the tensor.
// LDS: xs[nb] | xq[nb][8] | rows[8]
template <int kNit>
__device__ __forceinline__ void role_q80_rows(const Q80MatvecArgs& a, int tile, int tok, uint8_t* smem) {
  const int nb = a.in_dim >> 5, tid = threadIdx.x, nmat = a.w1 ? 2 : 1, RT = 8 / nmat;
  float* s_xs = (float*)smem;
  uint32_t* s_xq = (uint32_t*)(s_xs + align_up(nb, 4));
  float* s_rows = (float*)(s_xq + nb * 8);
  const int mat = nmat == 2 ? tid >> 7 : 0, rr = nmat == 2 ? (tid >> 5) & 3 : tid >> 5, l = tid & 31;
  const int row0 = tile * RT, row = min(row0 + rr, a.out_dim - 1);
  const uint8_t* wrow = (mat ? a.w1 : a.w0) + (size_t)row * nb * Q8_0_BYTES;
  const uint32_t sel = (l & 1) ? 0x07060504u : 0x05040302u, dsh = (l & 1) ? 16u : 0u;

  const uint32_t* xq = (const uint32_t*)(a.xq + (size_t)tok * nb * 32);
  const uint32_t* xs = (const uint32_t*)(a.xscale + (size_t)tok * nb);
  const int total = nb * 9;
  uint32_t sv[8];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int i = min(k * 256 + tid, total - 1);
    sv[k] = i < nb * 8 ? xq[i] : xs[i - nb * 8];
  }
  uint32_t wb[kNit][9];
#pragma unroll
  for (int i = 0; i < kNit; i++) {
    const int b_ = min(l + 32 * i, nb - 2 + (l & 1));
    const uint8_t* src_ = wrow + (size_t)b_ * Q8_0_BYTES - 2 * (l & 1);
    const uint4 v0 = *(const uint4*)src_, v1 = *(const uint4*)(src_ + 16);
    wb[i][0] = v0.x; wb[i][1] = v0.y; wb[i][2] = v0.z; wb[i][3] = v0.w;
    wb[i][4] = v1.x; wb[i][5] = v1.y; wb[i][6] = v1.z; wb[i][7] = v1.w;
    wb[i][8] = *(const uint32_t*)(src_ + 32);
  }
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int i = k * 256 + tid;
    if (i < nb * 8) s_xq[i] = sv[k];
    else if (i < total) ((uint32_t*)s_xs)[i - nb * 8] = sv[k];
  }
  for (int i = 2048 + tid; i < total; i += 256) {  // in_dim > 7280 only
    if (i < nb * 8) s_xq[i] = xq[i];
    else ((uint32_t*)s_xs)[i - nb * 8] = xs[i - nb * 8];
  }
  __syncthreads();

  float p = 0.0f;  // the reference's lane-strided partial l
#pragma unroll
  for (int i = 0; i < kNit; i++) {
    const int b = l + 32 * i;
    if (b < nb) {
      const uint4 qa = *(const uint4*)(s_xq + b * 8), qb = *(const uint4*)(s_xq + b * 8 + 4);
      const uint32_t qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
      int32_t d = 0;
#pragma unroll
      for (int k = 0; k < 8; k++) d = dot4(__builtin_amdgcn_perm(wb[i][k + 1], wb[i][k], sel), qv[k], d);
      const float sc = (float)__builtin_bit_cast(_Float16, (uint16_t)(wb[i][0] >> dsh));  // flushed: MODE
      p += sc * s_xs[b] * (float)d;
    }
  }
  p = group_sum<32>(p);
  if (l == 0) s_rows[mat * RT + rr] = p;
  __syncthreads();
  if (tid < RT && row0 + tid < a.out_dim) {
    const size_t off = (size_t)tok * a.out_dim + row0 + tid;
    if (nmat == 1) {
      a.out0[off] = s_rows[tid];
    } else {
      const float g0 = s_rows[tid], u0 = s_rows[RT + tid];
      if (a.out0) a.out0[off] = g0;
      if (a.out1) a.out1[off] = u0;
      if (a.mid) {  // device-coherent: a workgroup of this launch may quantize the group
        const float g = clamp_gate(g0, a.clamp), uu = clamp_up(u0, a.clamp);
        stc<true>(a.mid + off, (g / (1.0f + expf_dsm(-g))) * uu * 1.0f);
      }
    }
  }
}
__device__ __forceinline__ void role_q80_rows_any(const Q80MatvecArgs& a, int tile, int tok, uint8_t* smem) {
  switch ((a.in_dim + 1023) >> 10) {  // blocks per lane (in_dim <= 8192)
    case 1: role_q80_rows<1>(a, tile, tok, smem); break;
    case 2: role_q80_rows<2>(a, tile, tok, smem); break;
    case 3: role_q80_rows<3>(a, tile, tok, smem); break;
    case 4: role_q80_rows<4>(a, tile, tok, smem); break;
    case 5: role_q80_rows<5>(a, tile, tok, smem); break;
    case 6: role_q80_rows<6>(a, tile, tok, smem); break;
    case 7: role_q80_rows<7>(a, tile, tok, smem); break;
    default: role_q80_rows<8>(a, tile, tok, smem); break;
  }
}

struct DnItem {
  int s, rr, b;
  bool have;
};
__device__ __forceinline__ DnItem dn_item(const DownArgs& a, int row0, int it) {
  const int nb = a.I >> 8, per_slot = a.rows_per_wg * nb;
  DnItem q;
  q.s = it / per_slot;
  const int rem = it - q.s * per_slot;
  q.rr = rem / nb;
  q.b = rem - q.rr * nb;
  q.have = it < a.k * per_slot && row0 + q.rr < a.d;
  return q;
}
__device__ __forceinline__ void dn_load(const DownArgs& a, int e, int row0, const DnItem& q, uint32_t* wv) {
  if (!q.have) return;
  const size_t row_bytes = (size_t)(a.I >> 8) * Q2K_BYTES;
  const uint8_t* src = a.down + (size_t)e * a.d * row_bytes + (size_t)(row0 + q.rr) * row_bytes + (size_t)q.b * Q2K_BYTES;
#pragma unroll
  for (int j = 0; j < 5; j++) {
    const uint4 v4 = *(const uint4*)(src + 16 * j);
    wv[4 * j] = v4.x; wv[4 * j + 1] = v4.y; wv[4 * j + 2] = v4.z; wv[4 * j + 3] = v4.w;
  }
  wv[20] = *(const uint32_t*)(src + 80);
}
// One (row tile, token) unit of the down projection from preloaded weights.
template <bool kCoh>
__device__ __forceinline__ void dn_unit(const DownArgs& a, int tile, int tok, uint8_t* smem, const uint32_t* wv,
                                        bool stage) {
  const int nb = a.I >> 8, R = a.rows_per_wg, K = a.k, tid = threadIdx.x, B = blockDim.x;
  float* s_yd = (float*)smem;
  int16_t* s_bs = (int16_t*)(s_yd + align_up(K * nb, 4));
  uint8_t* s_q8 = (uint8_t*)(s_bs + K * nb * 16);
  float* s_vals = (float*)(s_q8 + K * nb * kQ8Stride);
  float* s_acc = s_vals + K * R * nb;
  const int row0 = tile * R;
  if (stage) stage_q8k<kCoh>(a.midq + (size_t)tok * K * nb * Q8K_BYTES, K * nb, s_q8, s_yd, s_bs);
  __syncthreads();
  const DnItem q = dn_item(a, row0, tid);
  if (q.have) {
    const int qb = q.s * nb + q.b;
    s_vals[(q.s * R + q.rr) * nb + q.b] = q2k_block_dot(wv, s_q8 + qb * kQ8Stride, s_bs + qb * 16, s_yd[qb]);
  }
  __syncthreads();
  for (int base = 0; base < K * R * 8; base += B) {
    const int t = base + tid;
    const int grp = t >> 3, l = t & 7;
    const int ss = grp / R, r2 = grp - ss * R;
    float p = (t < K * R * 8) ? lane_partial<8>(s_vals + (ss * R + r2) * nb, nb, l) : 0.0f;
    p = group_sum<8>(p);
    if (t < K * R * 8 && l == 0) {
      s_acc[ss * R + r2] = p;
      if (a.down_out && row0 + r2 < a.d) a.down_out[((size_t)tok * K + ss) * a.d + row0 + r2] = p;
    }
  }
  __syncthreads();
  if (a.out)
    for (int r2 = tid; r2 < R; r2 += B) {
      if (row0 + r2 >= a.d) continue;
      float total = 0.0f;
      for (int ss = 0; ss < K; ss++) total += s_acc[ss * R + r2];
      stc<kCoh>(a.out + (size_t)tok * a.d + row0 + r2, total);
    }
}


}  // namespace

// ===========================================================================
// Kernels
// ===========================================================================

// Router logits + Q8_K(x) + Q8_0(x) (blockDim 256): one router row, four
// Q8_K blocks or 32 Q8_0 blocks (8 when in_dim is not a multiple of 32) per
// workgroup.
// All threads: make this workgroup's coherent stores complete, then run `f`
// on thread 0 and broadcast its bool result.
template <class F>
__device__ __forceinline__ bool stores_done_then(int* s_flag, F f) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) *s_flag = f() ? 1 : 0;
  __syncthreads();
  return *s_flag != 0;
}

extern "C" __global__ __launch_bounds__(256) void dsmoe_prep(const PrepArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  int w = blockIdx.x;
  if (w < a.n_router) { role_router_logits<false>(a.router, w, smem); return; }
  w -= a.n_router;
  if (w < a.n_q8k) {
    if (q8k_waves_ok(a.q8k)) role_q8k_waves(a.q8k, w);
    else role_q8k<false, false>(a.q8k, w, smem);
    return;
  }
  w -= a.n_q8k;
  if (w < a.n_q80) {
    if (q80_waves_ok(a.q80)) role_q80_waves(a.q80, w);
    else role_q80<false, false>(a.q80, w, smem);
  }
}

// Routed + shared gate/up/SwiGLU.
// Workgroups [routed units][shared units].
extern "C" __global__ __launch_bounds__(1024) void dsmoe_up(const UpArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int n_gu = a.gu_tiles * a.gu_work;
  int w = blockIdx.x;
  if (w < n_gu) { role_gate_up<false>(a.gu, w % a.gu_tiles, w / a.gu_tiles, smem); return; }
  w -= n_gu;
  if (w < a.sh_tiles * a.sh_work) {
    if (a.sh_fmt == 0) role_q80_matvec<false>(a.sh_q80, w % a.sh_tiles, w / a.sh_tiles, smem);
    else role_gate_up<false>(a.sh_iq2, w % a.sh_tiles, w / a.sh_tiles, smem);
  }
}

// Routed gate/up in the row-streaming form (32 rows of one pair per
// workgroup) + the shared expert's workgroups.
__device__ __forceinline__ void role_gate_up_rows_any(const UpArgs& a, int tile, int pair, uint8_t* smem) {
  const RouterSelectArgs* rs = a.fuse_sel ? &a.sel : nullptr;
  switch ((a.gu.d + 1023) >> 10) {  // blocks per lane (d <= 8192)
    case 1: role_gate_up_rows<1>(a.gu, tile, pair, smem, rs); break;
    case 2: role_gate_up_rows<2>(a.gu, tile, pair, smem, rs); break;
    case 3: role_gate_up_rows<3>(a.gu, tile, pair, smem, rs); break;
    case 4: role_gate_up_rows<4>(a.gu, tile, pair, smem, rs); break;
    case 5: role_gate_up_rows<5>(a.gu, tile, pair, smem, rs); break;
    case 6: role_gate_up_rows<6>(a.gu, tile, pair, smem, rs); break;
    case 7: role_gate_up_rows<7>(a.gu, tile, pair, smem, rs); break;
    default: role_gate_up_rows<8>(a.gu, tile, pair, smem, rs); break;
  }
}

// With fuse_midq the quantization of the mid rows happens here too: each
// workgroup waits for its coherent mid stores, then counts its rows on the
// (pair, 256-row block) or (token, 256-row group) counter; the arrival that
// completes a counter resets it and quantizes that block (Q8_K,
// quantize.rs:309-417) or group (eight Q8_0 blocks, quantize.rs:147-225),
// reading the rows with coherent loads.  No workgroup waits for another.
extern "C" __global__ __launch_bounds__(256) void dsmoe_up_rows(const UpArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int s_flag;
  const int n_gu = a.gu_tiles * a.gu_work;
  int w = blockIdx.x;
  // f16 input denormals flushed while the rows are summed (the block scales'
  // widening is then one conversion, subnormals to signed zeros as in the
  // reference); restored before the mid quantization, whose f16 scales keep
  // their subnormal values
  __builtin_amdgcn_s_setreg(kHwregModeF16F64Denorm, 0);
  auto arrive = [&](uint32_t* c, uint32_t n, uint32_t target) {
    return stores_done_then(&s_flag, [&] {
      if (__hip_atomic_fetch_add(c, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + n != target) return false;
      __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return true;
    });
  };
  if (w < n_gu) {
    const int tile = w % a.gu_tiles, pair = w / a.gu_tiles;
    if (a.fuse_midq) {
      role_gate_up_rows_any(a, tile, pair, smem);
      __builtin_amdgcn_s_setreg(kHwregModeF16F64Denorm, kModeF16F64Preserve);
      const int nbI = a.gu.I >> 8, row0 = tile * 32, blk = row0 >> 8;
      const uint32_t n = (uint32_t)min(32, a.gu.I - row0), target = (uint32_t)min(256, a.gu.I - (blk << 8));
      if (arrive(a.mid_cnt + pair * nbI + blk, n, target) && threadIdx.x < 64) q8k_block_wave<true>(a.midq, pair * nbI + blk);
      return;
    }
    role_gate_up_rows_any(a, tile, pair, smem);
    return;
  }
  w -= n_gu;
  if (w < a.sh_tiles * a.sh_work) {
    const int tile = w % a.sh_tiles, tok = w / a.sh_tiles;
    if (a.sh_fmt == 0) {
      // With a large shared expert its workgroups start about 8 us (2 x 127
      // x 64 cycles) late: the routed workgroups first load the logits and
      // the activation words, which otherwise queue behind its stream (the
      // routing sits on the routed path, the shared rows do not).  Measured
      // per decode step at c2 (31 MB of shared gate/up): 53.4-53.9 us
      // without, 52.1-52.8 with this delay; 2, 4, 12 and 16 us were worse
      // or equal.  At c1 (6 MB) the delay only lengthens the launch
      // (29.0 against 30.6 us per step), so the host sets it by size.
      if (a.sh_delay) {
        __builtin_amdgcn_s_sleep(127);
        __builtin_amdgcn_s_sleep(127);
      }
      role_q80_rows_any(a.sh_q80, tile, tok, smem);
      __builtin_amdgcn_s_setreg(kHwregModeF16F64Denorm, kModeF16F64Preserve);
      if (a.fuse_midq) {
        const int Is = a.sh_q80.out_dim, RT = 4, ng = (Is + 255) >> 8, row0 = tile * RT, g = row0 >> 8;
        const uint32_t n = (uint32_t)min(RT, Is - row0), target = (uint32_t)min(256, Is - (g << 8));
        uint32_t* c = a.mid_cnt + a.gu_work * (a.gu.I >> 8) + tok * ng + g;
        // the group's eight Q8_0 blocks by wave 0 (blocks past the row are dead lanes)
        if (arrive(c, n, target) && threadIdx.x < 64) {
          const int nb32 = Is / 32;
          Q80Args q = a.sh_midq;
          q.rows = tok + 1;  // lanes past this row's blocks stay dead
          q80_blocks_wave<true>(q, tok * nb32 + 8 * g);
        }
      }
    } else {
      role_gate_up<false>(a.sh_iq2, tile, tok, smem);
    }
  }
}

// Q8_K of mid rows + Q8_0 of the shared mid (blockDim 256): four Q8_K blocks
// per workgroup, 32 Q8_0 blocks (8 when in_dim is not a multiple of 32).
extern "C" __global__ __launch_bounds__(256) void dsmoe_midq(const MidqArgs a) {
  __shared__ __align__(16) uint8_t smem[2 * 256 * 4 + 256];
  int w = blockIdx.x;
  if (w < a.n_a) {
    if (q8k_waves_ok(a.q8k_a)) role_q8k_waves(a.q8k_a, w);
    else role_q8k<false, false>(a.q8k_a, w, smem);
    return;
  }
  w -= a.n_a;
  if (w < a.n_b) {
    if (q8k_waves_ok(a.q8k_b)) role_q8k_waves(a.q8k_b, w);
    else role_q8k<false, false>(a.q8k_b, w, smem);
    return;
  }
  w -= a.n_b;
  if (w < a.n_q80) {
    if (q80_waves_ok(a.q80)) role_q80_waves(a.q80, w);
    else role_q80<false, false>(a.q80, w, smem);
  }
}

// Routed down + shared down.
extern "C" __global__ __launch_bounds__(1024) void dsmoe_dn(const DnArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int n_dn = a.dn_tiles * a.dn_work;
  int w = blockIdx.x;
  if (w < n_dn) { role_down<false>(a.dn, w % a.dn_tiles, w / a.dn_tiles, smem); return; }
  w -= n_dn;
  if (w < a.sh_tiles * a.sh_work) {
    if (a.sh_fmt == 0) role_q80_matvec<false>(a.sh_q80, w % a.sh_tiles, w / a.sh_tiles, smem);
    else role_down<false>(a.sh_q2k, w % a.sh_tiles, w / a.sh_tiles, smem);
  }
}

// Routed down (row-streaming form) + shared down (Q8_0 row-streaming form).
extern "C" __global__ __launch_bounds__(256) void dsmoe_dn_rows(const DnArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int n_dn = a.dn_tiles * a.dn_work;
  int w = blockIdx.x;
  // f16 input denormals flushed (the Q8_0 rows' scale widening; the launch
  // writes no f16)
  __builtin_amdgcn_s_setreg(kHwregModeF16F64Denorm, 0);
  if (w < n_dn) { role_down_rows_any(a.dn, w % a.dn_tiles, w / a.dn_tiles, smem); return; }
  w -= n_dn;
  if (w < a.sh_tiles * a.sh_work) {
    if (a.sh_fmt == 0) role_q80_rows_any(a.sh_q80, w % a.sh_tiles, w / a.sh_tiles, smem);
    else role_down<false>(a.sh_q2k, w % a.sh_tiles, w / a.sh_tiles, smem);
  }
}

// Expert-major gate/up and down (batches with few pairs per expert):
// workgroup = (row tile, dispatch chunk); chunks past the dispatch's count
// return at once.
extern "C" __global__ __launch_bounds__(256) void dsmoe_up_em(const GuEmArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  if (a.path && (*a.path & a.path_mask) != a.path_want) return;
  const int tile = blockIdx.x % a.tiles, chunk = blockIdx.x / a.tiles;
  if (chunk >= (int)a.tile_offsets[a.gu.E]) return;
  const int e = (int)a.tile_experts[chunk];
  const int p0 = (int)(a.offsets[e] + a.tile_starts[chunk]);
  const int cnt = min(a.np, (int)a.offsets[e + 1] - p0);
  switch ((a.gu.d + 1023) >> 10) {  // blocks per lane (d <= 8192)
    case 1: role_gate_up_em<1>(a, tile, e, p0, cnt, smem); break;
    case 2: role_gate_up_em<2>(a, tile, e, p0, cnt, smem); break;
    case 3: role_gate_up_em<3>(a, tile, e, p0, cnt, smem); break;
    case 4: role_gate_up_em<4>(a, tile, e, p0, cnt, smem); break;
    case 5: role_gate_up_em<5>(a, tile, e, p0, cnt, smem); break;
    case 6: role_gate_up_em<6>(a, tile, e, p0, cnt, smem); break;
    case 7: role_gate_up_em<7>(a, tile, e, p0, cnt, smem); break;
    default: role_gate_up_em<8>(a, tile, e, p0, cnt, smem); break;
  }
}

extern "C" __global__ __launch_bounds__(256) void dsmoe_dn_em(const DnEmArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  if (a.path && (*a.path & a.path_mask) != a.path_want) return;
  role_down_em(a, blockIdx.x % a.tiles, blockIdx.x / a.tiles, smem);
}


// Hash routing (moe.rs:92-109, weights :143-159), one workgroup per token:
// the probabilities of all experts, then thread 0 reads the token's row of
// the table and normalises the weights in slot order.
extern "C" __global__ __launch_bounds__(256) void dsmoe_router_select_hash(const HashSelectArgs a) {
  const int t = blockIdx.x, tid = threadIdx.x;
  if (a.probs)
    for (int e = tid; e < a.E; e += 256)
      a.probs[(size_t)t * a.E + e] = __builtin_sqrtf(softplus_dsm(a.logits[(size_t)t * a.E + e]));
  if (tid != 0) return;
  int tok = a.tokens ? a.tokens[t] : a.token_scalar;
  if (tok < 0 || tok >= a.hash_rows) tok = 0;
  float sum = 0.0f;
  for (int j = 0; j < a.k; j++) {
    const int e = a.hash[(size_t)tok * a.k + j];
    const float v = (e >= 0 && e < a.E) ? __builtin_sqrtf(softplus_dsm(a.logits[(size_t)t * a.E + e])) : 0.0f;
    a.selected[(size_t)t * a.k + j] = e;
    a.weights[(size_t)t * a.k + j] = v;
    sum += v;
  }
  if (sum < 6.103515625e-5f) sum = 6.103515625e-5f;
  for (int j = 0; j < a.k; j++) a.weights[(size_t)t * a.k + j] = a.weights[(size_t)t * a.k + j] / (sum / a.route_scale);
}

extern "C" __global__ __launch_bounds__(256) void dsmoe_router_select(const RouterSelectArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  role_select<false>(a, blockIdx.x, smem);
}

// utils.rs:141-163
extern "C" __global__ __launch_bounds__(256) void dsmoe_swiglu(const SwigluArgs a) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.n) return;
  const float g = clamp_gate(a.gate[i], a.clamp), u = clamp_up(a.up[i], a.clamp);
  a.out[i] = (g / (1.0f + expf_dsm(-g))) * u * a.weight;
}

// moe.rs:983-1005.  Four outputs per thread (16-byte loads) where
// moe_sum_vec_ok holds; each output is still the slot-ordered sum from 0.0f.
extern "C" __global__ __launch_bounds__(256) void dsmoe_moe_sum(const MoeSumArgs a) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (moe_sum_vec_ok(a)) {
    if (4 * i >= (size_t)a.T * a.d) return;
    const size_t tok = 4 * i / a.d, row = 4 * i % a.d;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (a.k <= 8) {
      // every slot's load in flight before the first add (each value is read
      // once: non-temporal); the adds stay in slot order from +0
      typedef float f4v __attribute__((ext_vector_type(4)));
      f4v v[8];
#pragma unroll
      for (int s = 0; s < 8; s++)
        if (s < a.k) v[s] = __builtin_nontemporal_load((const f4v*)(a.down + (tok * a.k + s) * a.d + row));
#pragma unroll
      for (int s = 0; s < 8; s++) {
        if (s < a.k) {
          acc.x = acc.x + v[s].x;
          acc.y = acc.y + v[s].y;
          acc.z = acc.z + v[s].z;
          acc.w = acc.w + v[s].w;
        }
      }
      *(float4*)(a.out + 4 * i) = acc;
      return;
    }
    for (int s = 0; s < a.k; s++) {
      const float4 v = *(const float4*)(a.down + (tok * a.k + s) * a.d + row);
      acc.x = acc.x + v.x;
      acc.y = acc.y + v.y;
      acc.z = acc.z + v.z;
      acc.w = acc.w + v.w;
    }
    *(float4*)(a.out + 4 * i) = acc;
    return;
  }
  if (i >= (size_t)a.T * a.d) return;
  const size_t tok = i / a.d, row = i % a.d;
  float acc = 0.0f;
  for (int s = 0; s < a.k; s++) acc += a.down[(tok * a.k + s) * a.d + row];
  a.out[i] = acc;
}

// norm.rs:14-63: thread tx sums the squares of elements tx, tx + 256, ...,
// the 128..1 halving tree in LDS, then every element times
// 1 / sqrt(sum / n + eps).
extern "C" __global__ __launch_bounds__(256) void dsmoe_rms_norm_plain(const RmsNormArgs a) {
  __shared__ float part[256];
  const int row = blockIdx.x, tx = threadIdx.x;
  const float* x = a.x + (size_t)row * a.n;
  float s = 0.0f;
  for (int i = tx; i < a.n; i += 256) s = s + x[i] * x[i];
  part[tx] = s;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (tx < st) part[tx] = part[tx] + part[tx + st];
    __syncthreads();
  }
  const float scale = 1.0f / __builtin_sqrtf(part[0] / (float)a.n + a.eps);
  for (int i = tx; i < a.n; i += 256) a.out[(size_t)row * a.n + i] = x[i] * scale;
}

// hc4_split_one (hc.rs:17-99) on one thread: pre weights, post weights and
// the Sinkhorn-normalised 4x4 comb of one row.
__device__ void hc4_split(const float* mix, const float* scale, const float* base, int iters, float eps,
                          float* out) {
  for (int i = 0; i < 4; i++) {
    const float z = mix[i] * scale[0] + base[i];
    out[i] = 1.0f / (1.0f + expf_dsm(-z)) + eps;
  }
  for (int i = 0; i < 4; i++) {
    const float z = mix[4 + i] * scale[1] + base[4 + i];
    out[4 + i] = 2.0f / (1.0f + expf_dsm(-z));
  }
  float c[16];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    float m = -__builtin_inff();
#pragma unroll
    for (int col = 0; col < 4; col++) {
      const float v = mix[8 + r * 4 + col] * scale[2] + base[8 + r * 4 + col];
      c[r * 4 + col] = v;
      if (v > m) m = v;
    }
    float s = 0.0f;
#pragma unroll
    for (int col = 0; col < 4; col++) {
      const float v = expf_dsm(c[r * 4 + col] - m);
      c[r * 4 + col] = v;
      s = s + v;
    }
#pragma unroll
    for (int col = 0; col < 4; col++) c[r * 4 + col] = c[r * 4 + col] / s + eps;
  }
  auto cols = [&]() {
#pragma unroll
    for (int col = 0; col < 4; col++) {
      float s = eps;
#pragma unroll
      for (int r = 0; r < 4; r++) s = s + c[r * 4 + col];
#pragma unroll
      for (int r = 0; r < 4; r++) c[r * 4 + col] = c[r * 4 + col] / s;
    }
  };
  cols();
  for (int it = 1; it < iters; it++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float s = eps;
#pragma unroll
      for (int col = 0; col < 4; col++) s = s + c[r * 4 + col];
#pragma unroll
      for (int col = 0; col < 4; col++) c[r * 4 + col] = c[r * 4 + col] / s;
    }
    cols();
  }
#pragma unroll
  for (int i = 0; i < 16; i++) out[8 + i] = c[i];
}

// hc.rs:313-398 (n_hc = 4): thread 0 writes the row's split, then thread tx
// forms out[i] = sum_h residual[h][i] * pre[h] for i = tx, tx + 256, ... and
// its squares, the 128..1 halving tree gives the norm, and
// norm_out[i] = out[i] * norm_scale * norm_w[i].
extern "C" __global__ __launch_bounds__(256) void dsmoe_hc_split_norm(const HcSplitNormArgs a) {
  __shared__ float part[256];
  __shared__ float sp[24];
  const int t = blockIdx.x, tx = threadIdx.x, n = a.n_embd;
  if (tx == 0) {
    hc4_split(a.mix + (size_t)t * 24, a.scale, a.base, a.iters, a.eps, sp);
    for (int i = 0; i < 24; i++) a.split[(size_t)t * 24 + i] = sp[i];
  }
  __syncthreads();
  const float* res = a.residual_hc + (size_t)t * 4 * n;
  float* o = a.out + (size_t)t * n;
  float s = 0.0f;
  for (int i = tx; i < n; i += 256) {
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < 4; h++) acc = acc + res[(size_t)h * n + i] * sp[h];
    o[i] = acc;
    s = s + acc * acc;
  }
  part[tx] = s;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (tx < st) part[tx] = part[tx] + part[tx + st];
    __syncthreads();
  }
  const float ns = 1.0f / __builtin_sqrtf(part[0] / (float)n + a.norm_eps);
  for (int i = tx; i < n; i += 256) a.norm_out[(size_t)t * n + i] = o[i] * ns * a.norm_w[i];
}

// hc.rs:212-259.  One thread per output element, or per four consecutive
// elements of one (token, destination stream) with 16-byte accesses; the
// split row is the same for a whole (token, destination) and comes from cache.
// Sums in the reference's order: (out (+ add)) * post, then + comb * residual
// for src = 0, 1, ... (no fused multiply-add).
extern "C" __global__ __launch_bounds__(256) void dsmoe_hc_expand(const HcExpandArgs a) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t per_tok = (size_t)a.n_hc * a.n_embd;
  const bool vec = hc_expand_vec_ok(a);
  const size_t e0 = vec ? 4 * i : i;
  if (e0 >= (size_t)a.T * per_tok) return;
  const size_t t = e0 / per_tok, rem = e0 % per_tok;
  const int dst = (int)(rem / a.n_embd), col = (int)(rem % a.n_embd);
  const float* row = a.split + t * a.mix_hc;
  const float post = row[a.n_hc + dst];
  const float* res = a.residual_hc + t * per_tok + col;
  if (vec) {
    float4 v = *(const float4*)(a.block_out + t * a.n_embd + col);
    if (a.has_add) {
      const float4 b = *(const float4*)(a.block_add + t * a.n_embd + col);
      v.x = v.x + b.x; v.y = v.y + b.y; v.z = v.z + b.z; v.w = v.w + b.w;
    }
    float4 acc = make_float4(v.x * post, v.y * post, v.z * post, v.w * post);
    for (int src = 0; src < a.n_hc; src++) {
      const float c = row[2 * a.n_hc + dst + src * a.n_hc];
      const float4 r = *(const float4*)(res + (size_t)src * a.n_embd);
      acc.x = acc.x + c * r.x; acc.y = acc.y + c * r.y; acc.z = acc.z + c * r.z; acc.w = acc.w + c * r.w;
    }
    *(float4*)(a.out_hc + e0) = acc;
    return;
  }
  float v = a.block_out[t * a.n_embd + col];
  if (a.has_add) v = v + a.block_add[t * a.n_embd + col];
  float acc = v * post;
  for (int src = 0; src < a.n_hc; src++) acc = acc + row[2 * a.n_hc + dst + src * a.n_hc] * res[(size_t)src * a.n_embd];
  a.out_hc[e0] = acc;
}

// ---------------------------------------------------------------------------
// Dispatch (moe.rs:299-362, :547-596) as one 1024-thread workgroup: per-wave
// expert histograms, an exclusive scan over (expert, wave), then a stable
// scatter where each wave walks its contiguous range of pairs in order.
// Within an expert the pairs are in ascending pair order.
// ---------------------------------------------------------------------------
namespace {
constexpr int kDispWaves = 16;
constexpr int kDispMaxE = 512;

__device__ __forceinline__ uint64_t peers_of(int e, bool live, int nbits) {
  uint64_t m = __ballot(live);
  for (int bit = 0; bit < nbits; bit++) {
    const uint64_t b = __ballot(live && ((e >> bit) & 1));
    m &= ((e >> bit) & 1) ? b : ~b;
  }
  return m;
}
}  // namespace

// Wave 0: out[i] = sum of f(in[j]) for j < i, out[n] = the total (n <=
// 512: eight entries per lane, then an inclusive scan over the lanes).
template <class F>
__device__ __forceinline__ void wave_exclusive_scan(const uint32_t* in, uint32_t* out, int n, F f) {
  const int lane = threadIdx.x & 63, per = (n + 63) >> 6;
  const int i0 = min(n, lane * per), i1 = min(n, i0 + per);
  uint32_t loc = 0;
  for (int i = i0; i < i1; i++) loc += f(in[i]);
  uint32_t incl = loc;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  uint32_t run = incl - loc;
  for (int i = i0; i < i1; i++) {
    const uint32_t c = f(in[i]);
    out[i] = run;
    run += c;
  }
  if (lane == 63) out[n] = incl;
}

extern "C" __global__ __launch_bounds__(1024) void dsmoe_dispatch(const DispatchArgs a) {
  __shared__ uint32_t s_cnt[kDispWaves][kDispMaxE];
  __shared__ uint32_t s_scan[kDispMaxE + 1];
  __shared__ uint32_t s_tot[kDispMaxE];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int E = a.E, P = a.pairs;
  int nbits = 0;
  while ((1 << nbits) < E) nbits++;
  for (int i = threadIdx.x; i < kDispWaves * kDispMaxE; i += blockDim.x) (&s_cnt[0][0])[i] = 0;
  __syncthreads();
  const int lo = (int)((long long)P * wv / kDispWaves), hi = (int)((long long)P * (wv + 1) / kDispWaves);
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  // the wave's expert ids are loaded kDispBatch chunks of 64 at a time (one
  // memory round trip per batch instead of per chunk)
  constexpr int kDispBatch = 16;
  auto load_ids = [&](int c0, int* ev) {
#pragma unroll
    for (int q = 0; q < kDispBatch; q++) {
      const int p = c0 + 64 * q + lane;
      int e = (c0 + 64 * q < hi && p < hi) ? a.selected[p] : 0;
      if (e < 0 || e >= E) e = 0;  // negative ids map to expert 0 (moe.rs:299-312); ids past E too
      ev[q] = e;
    }
  };
  for (int c0 = lo; c0 < hi; c0 += 64 * kDispBatch) {
    int ev[kDispBatch];
    load_ids(c0, ev);
#pragma unroll
    for (int q = 0; q < kDispBatch; q++) {
      if (c0 + 64 * q >= hi) break;  // wave-uniform: the rest of the batch is past the wave's range
      // counts need no order: one LDS atomic per pair (the ranks of the
      // scatter pass below keep the order)
      if (c0 + 64 * q + lane < hi) atomicAdd(&s_cnt[wv][ev[q]], 1u);
    }
  }
  __syncthreads();
  // totals per expert and per-(expert, wave) exclusive prefix
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    uint32_t run = 0;
    for (int w = 0; w < kDispWaves; w++) {
      const uint32_t c = s_cnt[w][e];
      s_cnt[w][e] = run;
      run += c;
    }
    s_tot[e] = run;
    a.counts[e] = run;
  }
  __syncthreads();
  if (wv == 0) wave_exclusive_scan(s_tot, s_scan, E, [](uint32_t c) { return c; });
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += blockDim.x) a.offsets[e] = s_scan[e];
  for (int e = threadIdx.x; e < E; e += blockDim.x)
    for (int w = 0; w < kDispWaves; w++) s_cnt[w][e] += s_scan[e];
  __syncthreads();
  for (int c0 = lo; c0 < hi; c0 += 64 * kDispBatch) {
    int ev[kDispBatch];
    load_ids(c0, ev);
#pragma unroll
    for (int q = 0; q < kDispBatch; q++) {
      if (c0 + 64 * q >= hi) break;
      const int p = c0 + 64 * q + lane, e = ev[q];
      const bool live = p < hi;
      const uint64_t pm = peers_of(e, live, nbits);
      if (live) {
        const uint32_t pos = s_cnt[wv][e] + (uint32_t)__popcll(pm & lt);
        a.sorted_pairs[pos] = (uint32_t)p;
      }
      __builtin_amdgcn_wave_barrier();
      if (live && (pm & lt) == 0) s_cnt[wv][e] += (uint32_t)__popcll(pm);
      __builtin_amdgcn_wave_barrier();
    }
  }
  auto tiles = [&](uint32_t bm, uint32_t* tile_offsets, uint32_t* tile_experts, uint32_t* tile_starts) {
    __syncthreads();
    if (wv == 0) wave_exclusive_scan(s_tot, s_scan, E, [bm](uint32_t c) { return (c + bm - 1) / bm; });
    __syncthreads();
    for (int e = threadIdx.x; e <= E; e += blockDim.x) tile_offsets[e] = s_scan[e];
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      const uint32_t n = (s_tot[e] + bm - 1) / bm;
      for (uint32_t t = 0; t < n; t++) {
        tile_experts[s_scan[e] + t] = (uint32_t)e;
        tile_starts[s_scan[e] + t] = t * bm;
      }
    }
    return s_scan[E];  // the tile count (every thread reads it before the next scan)
  };
  if (a.tile_offsets) {
    const uint32_t n1 = tiles((uint32_t)a.block_m, a.tile_offsets, a.tile_experts, a.tile_starts);
    if (a.tile_offsets2) {
      const uint32_t n2 = tiles((uint32_t)a.block_m2, a.tile_offsets2, a.tile_experts2, a.tile_starts2);
      // Expert-major (tiling 1) or grouped (tiling 2).  Measured on MI355X
      // (k = 8, E = 256, uniform and skewed loads): an expert-major chunk of
      // up to 4 pairs costs about 4/7 of a grouped 64-pair tile (c4: 376
      // chunks against 251 tiles, 0.84 against 0.97 ms of gate/up).
      if (a.path_flags && threadIdx.x == 0) {
        const uint32_t gu = 4u * n1 > 7u * n2 ? 1u : 0u;
        a.path_flags[0] = gu | ((gu || a.dn_grouped) ? 2u : 0u);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Synthetic tensors (test and benchmark data).  One thread per 256-element
// superblock (IQ2_XXS, Q2_K), per 32-element block (Q8_0) or per 256 plain
// elements (f16, f32).
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void dsmoe_synth(const SynthArgs a) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int per = (a.fmt == kSynQ80) ? 32 : 256;
  const int64_t bpr = (a.cols + per - 1) / per;
  const int64_t total = a.n_mats * a.rows * bpr;
  if (gid >= total) return;
  const int64_t mat = gid / (a.rows * bpr);
  const int64_t rem = gid - mat * a.rows * bpr;
  const int row = (int)(rem / bpr);
  const int blk = (int)(rem - (int64_t)row * bpr);
  const uint64_t key = tensor_key(a.seed, a.tensor_id);
  float x[256];
  const int c0 = blk * per;
  const int n = min(per, a.cols - c0);
#pragma clang loop unroll(disable)
  for (int i = 0; i < per; i++)
    x[i] = i < n ? synth_value(key, mat, row, c0 + i, a.rows_real, a.cols_real, a.sigma) : 0.0f;
  switch (a.fmt) {
    case kSynIq2xxs: iq2xxs_encode(x, a.out + gid * IQ2XXS_BYTES, a.lvlmap); break;
    case kSynQ2K: q2k_encode(x, a.out + gid * Q2K_BYTES); break;
    case kSynQ80: q8_0_encode(x, a.out + gid * Q8_0_BYTES); break;
    case kSynF16: {
      uint16_t* o = (uint16_t*)a.out + (mat * a.rows + row) * (int64_t)a.cols + c0;
#pragma clang loop unroll(disable)
      for (int i = 0; i < n; i++) o[i] = f32_to_f16_rne(x[i]);
      break;
    }
    default: {
      float* o = (float*)a.out + (mat * a.rows + row) * (int64_t)a.cols + c0;
#pragma clang loop unroll(disable)
      for (int i = 0; i < n; i++) o[i] = x[i];
      break;
    }
  }
}
