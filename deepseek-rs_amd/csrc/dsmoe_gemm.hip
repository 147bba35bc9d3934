// gfx950 grouped expert GEMMs of the MoE-FFN path for batches (prefill and
// batched decode).  Built as a second code object (dsmoe_gemm.hsaco) and
// loaded next to dsmoe_kernels.hsaco by dsmoe_host.cpp.
//
// Pairs (token, slot) are sorted by expert (dsmoe_dispatch) and cut into
// tiles of up to kGuBM pairs of one expert; a workgroup multiplies one tile
// by a slab of one expert's weight rows on the matrix cores.  The weights
// are dequantized per 256-element superblock into LDS as exact small
// integers in f16, the activations are the Q8_K integers in f16, and
// v_mfma_f32_32x32x16_f16 accumulates their products in f32.
//
// Exactness: every product is an integer of at most 24 bits and every
// partial sum of one superblock stays an integer below 2^24 (checked per
// superblock, below), so the f32 accumulator holds the reference's integer
// block sum exactly, in any summation order.  The per-superblock float
// epilogue and the sum over superblocks then follow the reference's order
// (lane-strided partials over 8 lanes, xor butterfly 4, 2, 1: moe.rs:35-41,
// :622-715), so results are bit-identical to the per-pair kernels.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "dsmoe_formats.h"
#include "dsmoe_kargs.h"
#include "dsmoe_math.h"

using namespace dsm;

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef int int16v __attribute__((ext_vector_type(16)));
// native 4-dword vector: arrays of it stay in registers (arrays of HIP's
// struct-wrapped uint4 are copied with memcpy and end up in scratch)
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Word 3 of a raw buffer descriptor on gfx9 (32-bit data format, no swizzle).
constexpr int kBufDword3 = 0x00020000;
constexpr int kRowH = 264;  // f16 per LDS operand row: 256 + 8 (528 B, 132 dwords = 4 mod 32 banks)
constexpr float kExactBound = 16777216.0f;  // 2^24

// Superblock visiting order: the reference's lane classes l = b mod 8 in the
// order its butterfly combines them, ((0+4)+(2+6)) + ((1+5)+(3+7)).
__device__ __forceinline__ int lane_class(int ci) {
  constexpr int order[8] = {0, 4, 2, 6, 1, 5, 3, 7};
  return order[ci];
}

// IQ2_XXS tables in LDS for dequantization to f16: the 8 grid magnitudes of
// each grid entry as f16 (exact small integers), their sum (for the
// exactness bound), and the sign pattern of each 7-bit sign index as 16-bit
// masks (0x8000 on the negative elements).
struct Iq2HalfTables {
  uint4 gridh[256];
  uint32_t gsum[256];
  uint4 sign[128];
};
__device__ __forceinline__ void load_iq2_half_tables(Iq2HalfTables* t) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  for (int i = threadIdx.x; i < 256; i += blockDim.x) {
    const uint64_t g = kIq2xxsGrid[i];
    uint32_t h[4], sum = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t lo = (uint32_t)(g >> (16 * j)) & 0xFF, hi = (uint32_t)(g >> (16 * j + 8)) & 0xFF;
      const h2 v = {(_Float16)(float)lo, (_Float16)(float)hi};
      h[j] = __builtin_bit_cast(uint32_t, v);
      sum += lo + hi;
    }
    t->gridh[i] = make_uint4(h[0], h[1], h[2], h[3]);
    t->gsum[i] = sum;
  }
  for (int i = threadIdx.x; i < 128; i += blockDim.x) {
    const uint32_t sb = iq2_sign_byte(i);
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
      w[j] = (((sb >> (2 * j)) & 1) ? 0x8000u : 0u) | (((sb >> (2 * j + 1)) & 1) ? 0x80000000u : 0u);
    t->sign[i] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}
// (g * ls) ^ sign for the 8 grid magnitudes g (f16 pairs): one f16 multiply
// per pair, exact (g * ls <= 43 * 31 = 1333 < 2048), then the sign bits.
__device__ __forceinline__ uint4 iq2_half8(uint4 gh, uint4 sgn, _Float16 ls) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 l2 = {ls, ls};
  auto cv = [&](uint32_t g2, uint32_t s) { return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, g2) * l2) ^ s; };
  return make_uint4(cv(gh.x, sgn.x), cv(gh.y, sgn.y), cv(gh.z, sgn.z), cv(gh.w, sgn.w));
}
// Folds the finished lane class cc (visiting position 0..7, see lane_class)
// into the butterfly tree ((p0+p4)+(p2+p6)) + ((p1+p5)+(p3+p7)); after
// cc = 7, h0 holds the row sum.
__device__ __forceinline__ void fold_class(int cc, const float16v& run, float16v& h0, float16v& h1, float16v& l2a) {
  switch (cc) {
    case 0: case 4: h0 = run; break;
    case 2: case 6: h1 = run; break;
    case 1: case 5:
      for (int i = 0; i < 16; i++) h0[i] = h0[i] + run[i];
      break;
    case 3:
      for (int i = 0; i < 16; i++) { h1[i] = h1[i] + run[i]; l2a[i] = h0[i] + h1[i]; }
      break;
    default:
      for (int i = 0; i < 16; i++) { h1[i] = h1[i] + run[i]; h0[i] = l2a[i] + (h0[i] + h1[i]); }
      break;
  }
}

// Number of superblocks of lane class position ci among nb.
__device__ __forceinline__ int class_len(int ci, int nb) {
  const int c = lane_class(ci);
  return c < nb ? (nb - c + 7) / 8 : 0;
}

// Work mapping for a 1-D grid of 8 * ceil(tiles / 8) * ny workgroups.  The
// dispatcher hands workgroup h to XCD h mod 8 (each XCD has its own L2).
// With at least 8 tiles each XCD gets a contiguous run of ceil(ntiles / 8)
// tiles: xcd_tile_slab puts all ny slabs of one tile back to back (the
// tile's activations are fetched into that XCD's L2 once and reused by every
// slab), xcd_slab_tile puts the slabs outermost (for dense GEMMs over a token
// batch a weight slab is then read once per XCD while the XCD's tiles of
// activations stay in its L2).  With fewer than 8 tiles that would leave
// XCDs idle, so the ntiles * ny items are cut into 8 equal runs instead.
// Any dispatch order still covers each (tile, slab) exactly once; only the
// cache reuse depends on it.  ntiles may be below the count the grid was
// sized for (the dispatch's tile count is read on the device): the extra
// workgroups return.
struct TileSlab {
  int t, n;
  bool ok;
};
__device__ __forceinline__ TileSlab xcd_items(int ntiles, int ny, bool slab_major) {
  const int h = blockIdx.x, xcd = h & 7, s = h >> 3;
  if (ntiles < 8) {
    const int W = ntiles * ny, per = (W + 7) >> 3, i = xcd * per + s;
    if (s >= per || i >= W) return {0, 0, false};
    return slab_major ? TileSlab{i % ntiles, i / ntiles, true} : TileSlab{i / ny, i % ny, true};
  }
  const int chunk = (ntiles + 7) >> 3;
  const int k = slab_major ? s % chunk : s / ny, n = slab_major ? s / chunk : s - (s / ny) * ny;
  const int t = xcd * chunk + k;
  return {t, n, n < ny && k < chunk && t < ntiles};
}
__device__ __forceinline__ TileSlab xcd_tile_slab(int ntiles, int ny) { return xcd_items(ntiles, ny, false); }
__device__ __forceinline__ TileSlab xcd_slab_tile(int ntiles, int ny) { return xcd_items(ntiles, ny, true); }

}  // namespace

// ---------------------------------------------------------------------------
// Routed gate/up/SwiGLU over sorted pairs (moe_gate_up_mid_sorted_qwarp32,
// moe.rs:721-815; per-pair arithmetic of moe.rs:622-715).  A workgroup of
// kGuThreads = 512 is one dispatch tile (up to kGuBM = 64 pairs of one expert)
// x kGuBN = 256 rows of gate and the same rows of up.  Wave w takes rows
// n0 + 32w .. +31 of gate and of up for all 64 pairs: four 32x32 MFMA tiles
// (pairs 0-31 / 32-63 x gate / up), so the SwiGLU needs no exchange between
// waves; with 8 waves (2 per SIMD) the activation tile serves 8 waves.
//
// A (the pairs' Q8_K integers as f16): one superblock (64 x 256) per LDS
// buffer, two buffers, loaded straight into LDS (global_load_lds_dwordx4):
// 16-byte chunk c of pair row m sits in slot m * 32 + (c ^ (m & 31)), so the
// operand reads (lanes = 32 rows x 2 chunks) are conflict-free.
// B (IQ2_XXS): lane l dequantizes its own weight row (l % 32) straight into
// the MFMA operand.  k-step ks of a superblock is group 2 (ks & 1) + l / 32 of
// sub-block ks / 2, i.e. eight consecutive weights, (g * ls) ^ sign as f16
// (exact small integers) from the grid / sign tables in LDS.  The row's 68
// raw bytes of a superblock are loaded one superblock ahead into registers.
// Both matrices of a wave share each A operand read, and each dequantized B
// operand serves both pair tiles.
//
// Per superblock each (pair, row) sum of integer products accumulates in f32
// on the matrix cores (exact while below 2^24); its block value
// 0.125 * xd * yd * sum is formed as in the reference and added to the
// row's running sum in superblock order 0, 1, 2, ...  The reference adds the
// blocks b = l mod 8 per lane l and then a butterfly over the 8 lanes, so the
// two agree to f32 rounding of that sum order (the integer and indexing work
// is the reference's exactly).
// ---------------------------------------------------------------------------
namespace {
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

// 68 bytes from a 4-byte aligned address (four 16-byte loads and a dword)
__device__ __forceinline__ void load17(const uint8_t* p, uint32_t* r) {
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const u32x4 v = *(const u32x4*)(p + 16 * q);
    r[4 * q] = v.x; r[4 * q + 1] = v.y; r[4 * q + 2] = v.z; r[4 * q + 3] = v.w;
  }
  r[16] = *(const uint32_t*)(p + 64);
}
}  // namespace

extern "C" __global__ __launch_bounds__(kGuThreads)
void dsmoe_gu_grouped(const GuGroupedArgs a) {
  __shared__ __align__(16) u32x4 sA[2][kGuBM * 32];
  __shared__ __align__(16) float s_yd[2][kGuBM];
  __shared__ Iq2HalfTables tab;
  // the f16 grid table in 16 copies, entry g of copy p at 16 g + p: the 16
  // lanes of one LDS pass (lane % 16 = p) each read their own bank group
  __shared__ u32x4 s_grid16[256 * 16];
  // the sign masks in 8 copies (entry i of copy p at 8 i + p, p = lane % 8)
  __shared__ u32x4 s_sign8[128 * 8];
  __shared__ uint32_t s_pair[kGuBM], s_xrow[kGuBM], s_qrow[kGuBM];

  const TileSlab ts = xcd_tile_slab((int)a.tile_offsets[a.E], a.I / kGuBN);
  if (!ts.ok) return;
  const int t = ts.t;
  const int e = (int)a.tile_experts[t];
  const int p0 = (int)(a.offsets[e] + a.tile_starts[t]);
  const int cnt = min(kGuBM, (int)a.offsets[e + 1] - p0);
  const int n0 = ts.n * kGuBN;
  const int tid = threadIdx.x, lane = tid & 63, kh = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar
  const int d = a.d, nb = d >> 8, I = a.I, K = a.k;

  if (tid < kGuBM) {
    const uint32_t pr = tid < cnt ? a.sorted_pairs[p0 + tid] : 0xFFFFFFFFu;
    const uint32_t tok = pr != 0xFFFFFFFFu ? pr / (uint32_t)K : 0u;  // dead rows read token 0, never stored
    s_pair[tid] = pr;
    s_xrow[tid] = tok * (uint32_t)d * 2u;
    s_qrow[tid] = tok * (uint32_t)nb * (uint32_t)Q8K_BYTES;
  }
  load_iq2_half_tables(&tab);
  __syncthreads();
  for (int i = tid; i < 256 * 16; i += kGuThreads) {
    const uint4 g = tab.gridh[i >> 4];
    s_grid16[i] = u32x4{g.x, g.y, g.z, g.w};
  }
  __syncthreads();
  for (int i = tid; i < 128 * 8; i += kGuThreads) {
    const uint4 g = tab.sign[i >> 3];
    s_sign8[i] = u32x4{g.x, g.y, g.z, g.w};
  }
  __syncthreads();
  const u32x4* grid16 = &s_grid16[lane & 15];
  const u32x4* sign8 = &s_sign8[lane & 7];

  // A: wave w's loads per superblock fill slots (kAj w + j) * 64 + lane
  constexpr int kAj = 2048 / 64 / (kGuThreads / 64);
  uint32_t aoff[kAj];
#pragma unroll
  for (int j = 0; j < kAj; j++) {
    const int sl = (kAj * w + j) * 64 + lane, m = sl >> 5, c = (sl & 31) ^ (m & 31);
    aoff[j] = s_xrow[m] + 16u * (uint32_t)c;
  }
  const uint32_t qoff = s_qrow[lane];
  auto issue_a = [&](int b, int buf) {
    const uint8_t* base = (const uint8_t*)a.xh + 512 * b;
#pragma unroll
    for (int j = 0; j < kAj; j++)
      __builtin_amdgcn_global_load_lds((glb_void*)(base + aoff[j]), (lds_void*)&sA[buf][(kAj * w + j) * 64], 16, 0, 0);
    if (w == 0)  // the 64 pairs' block scales: lane l -> s_yd[buf][l]
      __builtin_amdgcn_global_load_lds((glb_void*)(a.xq + qoff + (size_t)b * Q8K_BYTES), (lds_void*)&s_yd[buf][0], 4,
                                       0, 0);
  };
  const size_t rb = (size_t)nb * IQ2XXS_BYTES;
  const size_t row = (size_t)e * I + n0 + 32 * w + l32;
  const uint8_t* grow = a.gate + row * rb;
  const uint8_t* urow = a.up + row * rb;
  // superblock b's 68 bytes from its dword-aligned start (odd b: 2 bytes before)
  auto raw_at = [&](const uint8_t* r, int b) { return r + IQ2XXS_BYTES * b - 2 * (b & 1); };

  float16v rg0, rg1, ru0, ru1;  // running sums: pairs 0-31 / 32-63 x gate / up
#pragma unroll
  for (int i = 0; i < 16; i++) { rg0[i] = 0.0f; rg1[i] = 0.0f; ru0[i] = 0.0f; ru1[i] = 0.0f; }

  // one superblock from LDS buffer buf and raw rows gr / ur (kEven: the qs
  // start 2 bytes into the loaded words)
  auto superblock = [&](auto even_tag, int buf, uint32_t* gr, uint32_t* ur) {
    constexpr bool kEven = decltype(even_tag)::value;
    // the block scale, then the qs words realigned in place (even superblocks
    // start 2 bytes into the loaded words): qs word j is r[j + 1]
    const uint32_t dg = kEven ? gr[0] & 0xFFFF : gr[0] >> 16, du = kEven ? ur[0] & 0xFFFF : ur[0] >> 16;
    if (kEven) {
#pragma unroll
      for (int j = 0; j < 16; j++) {
        gr[j] = __builtin_amdgcn_alignbyte(gr[j + 1], gr[j], 2);
        ur[j] = __builtin_amdgcn_alignbyte(ur[j + 1], ur[j], 2);
      }
    }
    auto qs = [&](const uint32_t* r, int j) -> uint32_t { return kEven ? r[j] : r[j + 1]; };
    float16v ag0, ag1, au0, au1;
#pragma unroll
    for (int i = 0; i < 16; i++) { ag0[i] = 0.0f; ag1[i] = 0.0f; au0[i] = 0.0f; au1[i] = 0.0f; }
    _Float16 lsg = 1, lsu = 1;
    uint32_t g1 = 0, u1 = 0;
    const u32x4* sa = &sA[buf][0];
#pragma unroll
    for (int ks = 0; ks < 16; ks++) {
      const int sb = ks >> 1;
      if ((ks & 1) == 0) {
        g1 = qs(gr, 2 * sb + 1);
        u1 = qs(ur, 2 * sb + 1);
        lsg = (_Float16)(float)(2 * (g1 >> 28) + 1);
        lsu = (_Float16)(float)(2 * (u1 >> 28) + 1);
      }
      const uint32_t sh0 = 16 * (ks & 1) + 8 * kh, sh1 = 14 * (ks & 1) + 7 * kh;
      const uint32_t gg = __builtin_amdgcn_ubfe(qs(gr, 2 * sb), sh0, 8), gs = __builtin_amdgcn_ubfe(g1, sh1, 7);
      const uint32_t ug = __builtin_amdgcn_ubfe(qs(ur, 2 * sb), sh0, 8), us = __builtin_amdgcn_ubfe(u1, sh1, 7);
      const u32x4 gv = grid16[16 * gg], uv = grid16[16 * ug];
      const u32x4 gsv = sign8[8 * gs], usv = sign8[8 * us];
      const half8 bg = __builtin_bit_cast(half8, iq2_half8(make_uint4(gv.x, gv.y, gv.z, gv.w),
                                                           make_uint4(gsv.x, gsv.y, gsv.z, gsv.w), lsg));
      const half8 bu = __builtin_bit_cast(half8, iq2_half8(make_uint4(uv.x, uv.y, uv.z, uv.w),
                                                           make_uint4(usv.x, usv.y, usv.z, usv.w), lsu));
      const int c = (2 * ks + kh) ^ l32;
      const half8 a0 = __builtin_bit_cast(half8, sa[l32 * 32 + c]);
      const half8 a1 = __builtin_bit_cast(half8, sa[(32 + l32) * 32 + c]);
      ag0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, bg, ag0, 0, 0, 0);
      au0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, bu, au0, 0, 0, 0);
      ag1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, bg, ag1, 0, 0, 0);
      au1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, bu, au1, 0, 0, 0);
    }
    // block values 0.125 * xd * yd * sum (quantize.rs:763-812), added in superblock order
    const float cg = 0.125f * f16_to_f32_ftz((uint16_t)dg);
    const float cu = 0.125f * f16_to_f32_ftz((uint16_t)du);
    const float* yd = &s_yd[buf][0];
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const int m = 8 * (k >> 2) + 4 * kh + (k & 3);
      const float y0 = yd[m], y1 = yd[32 + m];
      rg0[k] = __builtin_fmaf(cg * y0, ag0[k], rg0[k]);
      ru0[k] = __builtin_fmaf(cu * y0, au0[k], ru0[k]);
      rg1[k] = __builtin_fmaf(cg * y1, ag1[k], rg1[k]);
      ru1[k] = __builtin_fmaf(cu * y1, au1[k], ru1[k]);
    }
  };

  uint32_t gE[17], uE[17], gO[17], uO[17];
  load17(raw_at(grow, 0), gE);
  load17(raw_at(urow, 0), uE);
  issue_a(0, 0);
  for (int b = 0; b < nb; b += 2) {  // nb is even (d is a multiple of 512)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    issue_a(b + 1, 1);
    load17(raw_at(grow, b + 1), gO);
    load17(raw_at(urow, b + 1), uO);
    superblock(std::true_type{}, 0, gE, uE);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (b + 2 < nb) {
      issue_a(b + 2, 0);
      load17(raw_at(grow, b + 2), gE);
      load17(raw_at(urow, b + 2), uE);
    }
    superblock(std::false_type{}, 1, gO, uO);
  }

  // SwiGLU (utils.rs:141-163) and the routing weight; rows of dead pairs are not stored
#pragma unroll
  for (int mt = 0; mt < 2; mt++) {
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const int m = 32 * mt + 8 * (k >> 2) + 4 * kh + (k & 3);
      if (m >= cnt) continue;
      const uint32_t pair = s_pair[m];
      const float g = clamp_gate(mt ? rg1[k] : rg0[k], a.clamp), u = clamp_up(mt ? ru1[k] : ru0[k], a.clamp);
      const float wgt = a.weights ? a.weights[pair] : 1.0f;
      a.mid[(size_t)pair * I + n0 + 32 * w + l32] = (g / (1.0f + expf_dsm(-g))) * u * wgt;
    }
  }
}

// ---------------------------------------------------------------------------
// Routed down projection over sorted pairs (moe_down_sorted_qwarp32 /
// moe_down_qwarp32, moe.rs:821-916; block arithmetic quantize.rs:846-901).
// Per superblock: isum = sum_k (sc_lo * q)[n][k] * q8[m][k] (weights 0..45 in
// f16, |isum| < 2^21) and summs = sum_j bsums[m][j] * sc_hi[n][j] (a K = 16
// product), both exact in f32; then dall * isum - dmin' * summs with
// dall = yd * d, dmin' = yd * dmin, and the per-pair row sum over
// superblocks in the reference's 8-lane order.  The slot sum is moe_sum.
// grid = 8 * ceil(max tiles / 8) * (d / kDnBN) (xcd_tile_slab), 256 threads: wave w computes pairs
// 32*(w&1).. x rows 32*(w>>1)..
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void dsmoe_dn_grouped(const DnGroupedArgs a) {
  // A: row-major [pair][32 chunks], chunk XOR-swizzled by (row & 15)
  // B: chunk-major [32 chunks][64 rows], row slot XOR-swizzled by 2 * (chunk / 8)
  __shared__ uint4 sA[kGuBM][32];
  __shared__ uint4 sB[32][kDnBN];
  __shared__ __align__(16) _Float16 sBS[kGuBM][16];  // bsums
  __shared__ __align__(16) _Float16 sM[kDnBN][16];   // sc >> 4
  __shared__ float s_yd[kGuBM], s_d[kDnBN], s_dmin[kDnBN];
  __shared__ uint32_t s_pair[kGuBM];

  const TileSlab ts = xcd_tile_slab((int)a.tile_offsets[a.E], a.d / kDnBN);
  if (!ts.ok) return;
  const int t = ts.t;
  const int e = (int)a.tile_experts[t];
  const int p0 = (int)(a.offsets[e] + a.tile_starts[t]);
  const int cnt = min(kGuBM, (int)a.offsets[e + 1] - p0);
  const int n0 = ts.n * kDnBN;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int d = a.d, I = a.I, nb = I >> 8;

  if (tid < kGuBM) s_pair[tid] = tid < cnt ? a.sorted_pairs[p0 + tid] : 0xFFFFFFFFu;
  __syncthreads();

  // Wave w owns rows 16w .. 16w+15 of both operands; lane l handles row
  // 16w + l/4, quarter p = l % 4 (elements 64p .. 64p+63 of a superblock).
  // Dead pair rows read pair 0: finite, never stored.
  const int r = 16 * w + (lane >> 2), pq = lane & 3;
  // activation loads: instruction j covers rows 16w + 2j + lane/32, chunk lane % 32
  uint32_t aoff[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t pr = s_pair[16 * w + 2 * j + (lane >> 5)];
    aoff[j] = (pr != 0xFFFFFFFFu ? pr : 0u) * (uint32_t)I + 8 * (lane & 31);
  }
  const uint32_t mpair = s_pair[r] != 0xFFFFFFFFu ? s_pair[r] : 0u;
  const uint8_t* mrow = a.mq + (size_t)mpair * nb * Q8K_BYTES;
  const uint8_t* wrow = a.down + ((size_t)e * d + n0 + r) * nb * Q2K_BYTES;

  // named registers: an array captured by the lambdas ends up in scratch
  uint4 av0, av1, av2, av3, av4, av5, av6, av7;
  uint32_t abs0, abs1, bsc, bdd;
  uint4 bq0, bq1;
  float ayd;
  auto issue = [&](int b) {
    const uint16_t* base = a.mh + 256 * b;
    av0 = *(const uint4*)(base + aoff[0]);
    av1 = *(const uint4*)(base + aoff[1]);
    av2 = *(const uint4*)(base + aoff[2]);
    av3 = *(const uint4*)(base + aoff[3]);
    av4 = *(const uint4*)(base + aoff[4]);
    av5 = *(const uint4*)(base + aoff[5]);
    av6 = *(const uint4*)(base + aoff[6]);
    av7 = *(const uint4*)(base + aoff[7]);
    const uint8_t* mb = mrow + (size_t)b * Q8K_BYTES;
    ayd = ld_f32(mb);
    abs0 = *(const uint32_t*)(mb + 260 + 8 * pq);
    abs1 = *(const uint32_t*)(mb + 264 + 8 * pq);
    const uint32_t* blk = (const uint32_t*)(wrow + (size_t)b * Q2K_BYTES);
    bsc = blk[pq];                                      // scales of groups 4p .. 4p+3
    bq0 = *(const uint4*)(blk + 4 + 8 * (pq >> 1));     // qs half p / 2 (32 bytes)
    bq1 = *(const uint4*)(blk + 8 + 8 * (pq >> 1));
    bdd = blk[20];                                      // d | dmin
  };
  auto commit = [&]() {
#define DSM_STORE_A(j, v)                            \
    {                                                \
      const int row = 16 * w + 2 * (j) + (lane >> 5); \
      sA[row][(lane & 31) ^ (row & 15)] = v;         \
    }
    DSM_STORE_A(0, av0)
    DSM_STORE_A(1, av1)
    DSM_STORE_A(2, av2)
    DSM_STORE_A(3, av3)
    DSM_STORE_A(4, av4)
    DSM_STORE_A(5, av5)
    DSM_STORE_A(6, av6)
    DSM_STORE_A(7, av7)
#undef DSM_STORE_A
    {
      typedef _Float16 h4 __attribute__((ext_vector_type(4)));
      const h4 v = {(_Float16)(float)(int16_t)(abs0 & 0xFFFF), (_Float16)(float)(int16_t)(abs0 >> 16),
                    (_Float16)(float)(int16_t)(abs1 & 0xFFFF), (_Float16)(float)(int16_t)(abs1 >> 16)};
      *(h4*)&sBS[r][4 * pq] = v;
      const h4 m = {(_Float16)(float)((bsc >> 4) & 0xF), (_Float16)(float)((bsc >> 12) & 0xF),
                    (_Float16)(float)((bsc >> 20) & 0xF), (_Float16)(float)((bsc >> 28) & 0xF)};
      *(h4*)&sM[r][4 * pq] = m;
    }
    if (pq == 0) {
      s_yd[r] = ayd;
      s_d[r] = f16_to_f32_ftz((uint16_t)(bdd & 0xFFFF));
      s_dmin[r] = f16_to_f32_ftz((uint16_t)(bdd >> 16));
    }
    const uint32_t bqs[8] = {bq0.x, bq0.y, bq0.z, bq0.w, bq1.x, bq1.y, bq1.z, bq1.w};
    const int slot = r ^ (2 * pq);
    // weights sc_lo * q as f16: each group's values {0, L, 2L, 3L} are a
    // 4-entry table that v_perm indexes with the 2-bit codes
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++) {
      const uint32_t shift = 2 * (2 * (pq & 1) + s2);
#pragma unroll
      for (int gh = 0; gh < 2; gh++) {  // the two 16-element groups of this 32-element run
        const uint32_t L = (bsc >> (8 * (2 * s2 + gh))) & 0xF;
        const uint32_t t_lo = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)L) << 16;
        const uint32_t t_hi = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)(2 * L)) |
                              ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)(3 * L)) << 16);
        uint32_t o[8];
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
          const uint32_t qb = (bqs[4 * gh + tt] >> shift) & 0x03030303u;
          const uint32_t x01 = __builtin_amdgcn_perm(0u, qb, 0x0c010c00u), x23 = __builtin_amdgcn_perm(0u, qb, 0x0c030c02u);
          o[2 * tt] = __builtin_amdgcn_perm(t_hi, t_lo, x01 * 0x0202u + 0x01000100u);
          o[2 * tt + 1] = __builtin_amdgcn_perm(t_hi, t_lo, x23 * 0x0202u + 0x01000100u);
        }
        const int c = 8 * pq + 4 * s2 + 2 * gh;  // elements 8c .. 8c+15
        sB[c][slot] = make_uint4(o[0], o[1], o[2], o[3]);
        sB[c + 1][slot] = make_uint4(o[4], o[5], o[6], o[7]);
      }
    }
  };

  const int mt = w & 1, nt = w >> 1, hh = lane >> 5;
  const int arow_l = mt * 32 + (lane & 31), brow_l = nt * 32 + (lane & 31), koff = 8 * hh;
  float16v run, h0, h1, l2a;
  for (int i = 0; i < 16; i++) { run[i] = 0.0f; h0[i] = 0.0f; h1[i] = 0.0f; l2a[i] = 0.0f; }
  auto block_of = [&](int ci, int j) { return lane_class(ci) + 8 * j; };

  int ci = 0;
  while (ci < 8 && class_len(ci, nb) == 0) ci++;
  if (ci < 8) issue(block_of(ci, 0));
  for (int cc = 0; cc < 8; cc++) {
    const int len = class_len(cc, nb);
    for (int jj = 0; jj < len; jj++) {
      __syncthreads();
      commit();
      // the next superblock's loads (unconditional: past the end re-reads
      // superblock 0, never used; keeps the wait counts exact)
      int nc = cc, nj = jj + 1;
      if (nj >= len) {
        nc = cc + 1;
        nj = 0;
        while (nc < 8 && class_len(nc, nb) == 0) nc++;
      }
      issue(nc < 8 ? block_of(nc, nj) : 0);
      __syncthreads();
      float16v isum, summs;
      for (int i = 0; i < 16; i++) { isum[i] = 0.0f; summs[i] = 0.0f; }
#pragma unroll
      for (int ks = 0; ks < 16; ks++) {
        const int c = 2 * ks + hh;
        const half8 av8 = *(const half8*)&sA[arow_l][c ^ (arow_l & 15)];
        const half8 bv8 = *(const half8*)&sB[c][brow_l ^ (2 * (ks >> 2))];
        isum = __builtin_amdgcn_mfma_f32_32x32x16_f16(av8, bv8, isum, 0, 0, 0);
      }
      summs = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const half8*)&sBS[arow_l][koff],
                                                      *(const half8*)&sM[brow_l][koff], summs, 0, 0, 0);
      const float dn = s_d[brow_l], dm = s_dmin[brow_l];
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int m = mt * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
        const float yd = s_yd[m];
        const float dall = yd * dn, dmin = yd * dm;
        run[i] = run[i] + (dall * isum[i] - dmin * summs[i]);
      }
    }
    fold_class(cc, run, h0, h1, l2a);
    for (int i = 0; i < 16; i++) run[i] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int m = mt * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
    if (m >= cnt) continue;
    a.down_out[(size_t)s_pair[m] * d + n0 + nt * 32 + (lane & 31)] = h0[i];
  }
}

// ---------------------------------------------------------------------------
// Shared expert for batches: Q8_0 weights x Q8_0 activations
// (matmul_q8_0_preq_batch_warp8, matmul.rs:412-458; row arithmetic of
// matmul_q8_0_preq_warp8, matmul.rs:357-405; swiglu utils.rs:141-163).
// Per 32-element block: sumi = sum of 32 code products (|sumi| < 2^19, exact
// in f32 through two K = 16 MFMAs), v = (d_w * d_x) * sumi; a row is the
// 32-lane strided sum over blocks followed by the 16, 8, 4, 2, 1 halving
// tree, reproduced by visiting the blocks lane class by lane class in
// bit-reversed order and folding the classes like a binary counter.
// grid = 8 * ceil(ceil(T / 64) / 8) * out_dim / (kSwiglu ? 32 : 64)
// (xcd_slab_tile), 256 threads.
// ---------------------------------------------------------------------------
namespace {

__device__ __forceinline__ int bitrev5(int k) {
  return ((k & 1) << 4) | ((k & 2) << 2) | (k & 4) | ((k & 8) >> 2) | ((k & 16) >> 4);
}

// int8 codes (4 per dword) -> f16 (2 per dword): (b ^ 0x80) as the mantissa
// of 1024 + b' is exact; subtracting 1152 leaves the signed code.
__device__ __forceinline__ void i8x4_to_f16(uint32_t v, uint32_t& lo, uint32_t& hi) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const uint32_t u = v ^ 0x80808080u;
  const h2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u, 0x05010400u)) + bias);
  hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u, 0x07030602u)) + bias);
}

}  // namespace

// A: row-major [token][32 chunks] (chunk 4u + p = elements 8p .. 8p+7 of
//    stage slot u), chunk XOR-swizzled by (row & 15)
// B: chunk-major [32 chunks][64 weight rows]
struct Q80Smem {
  uint4 sA[kGuBM][32];
  uint4 sB[32][64];
  float s_xs[8][kGuBM], s_sw[64][8];  // s_xs by slot: four consecutive tokens per read
};

// kJ = blocks per lane class, ceil(nb / 32), as a compile-time constant (0:
// taken from in_dim at run time).
template <bool kSwiglu, int kJ>
__device__ __forceinline__ void q80_gemm(const Q80GemmArgs& a, Q80Smem& sm) {
  auto& sA = sm.sA;
  auto& sB = sm.sB;
  auto& s_xs = sm.s_xs;
  auto& s_sw = sm.s_sw;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int in = a.in_dim, nb = in >> 5, T = a.T;
  const int S = a.ksplit;
  const TileSlab ts = xcd_slab_tile((T + kGuBM - 1) / kGuBM, a.out_dim / (kSwiglu ? 32 : 64) * S);
  if (!ts.ok) return;
  const int m0 = ts.t * kGuBM;
  const int n0 = (ts.n / S) * (kSwiglu ? 32 : 64), split = ts.n % S;
  const int kb = split * (32 / S), ke = kb + 32 / S;  // class positions of this workgroup

  // A stage holds up to 8 blocks: G = 8 / jmax lane classes of jmax slots
  // each (jmax = blocks of the longest class); slot u = class position
  // k0 + u / jmax, member u % jmax (empty when past that class's length).
  const int jmax = kJ ? kJ : (nb + 31) >> 5;
  const int G = 8 / jmax;
  auto nblk = [&](int l) { return l < nb ? (nb - l + 31) / 32 : 0; };

  // lane l: row 16w + (l & 15), chunk p = l >> 4 of each block
  const int r = 16 * w + (lane & 15), p = lane >> 4;
  const int tok = min(m0 + r, T - 1);  // rows past T re-read the last token (never stored)
  const uint16_t* arow = a.xh + (size_t)tok * in + 8 * p;
  const float* xsrow = a.xs + (size_t)tok * nb;
  const uint8_t* wrow = kSwiglu ? ((r < 32 ? a.w0 : a.w1) + (size_t)(n0 + (r & 31)) * nb * Q8_0_BYTES)
                                : (a.w0 + (size_t)(n0 + r) * nb * Q8_0_BYTES);

  // prefetch registers of one stage (8 slots).  The loads and stores are
  // macros over these local arrays: fully unrolled with constant indices
  // they stay in registers (arrays captured by a lambda end up in scratch).
  // 12-byte code window: one dwordx3 load (4-byte aligned)
  struct W3 {
    uint32_t x, y, z;
  };
  u32x4 av[8];
  W3 bc[8];
  uint32_t bd[2];  // weight block scales of slots p and p + 4 (this lane's share)
  float axs[2];    // activation block scales of slots p and p + 4
  auto slot_block = [&](int k0, int u) {
    const int k = k0 + u / jmax, j = u % jmax;
    if (k >= 32) return -1;
    const int l = bitrev5(k);
    return j < nblk(l) ? l + 32 * j : -1;
  };
#define DSM_Q80_ISSUE(K0)                                                            \
  _Pragma("clang loop unroll(full)") for (int u = 0; u < 8; u++) {                    \
    const int b0_ = slot_block((K0), u), b_ = b0_ < 0 ? 0 : b0_; /* empty: block 0 */ \
    av[u] = *(const u32x4*)(arow + 32 * b_);                                         \
    const uint8_t* blk_ = wrow + (size_t)b_ * Q8_0_BYTES;                            \
    /* codes 8p .. 8p+7 inside an aligned 12-byte window whose every dword */       \
    /* holds bytes of the tensor: [cs-2, cs+10) or [cs-4, cs+8) */                  \
    const uint8_t* cs_ = blk_ + 2 + 8 * p;                                           \
    __builtin_memcpy(&bc[u], cs_ - (((uintptr_t)cs_ & 3) ? 2 : 4), 12);              \
  }                                                                                  \
  _Pragma("clang loop unroll(full)") for (int h = 0; h < 2; h++) {                    \
    const int b0_ = slot_block((K0), p + 4 * h), b_ = b0_ < 0 ? 0 : b0_;             \
    axs[h] = xsrow[b_];                                                              \
    const uint8_t* blk_ = wrow + (size_t)b_ * Q8_0_BYTES;                            \
    bd[h] = *(const uint32_t*)(blk_ - ((uintptr_t)blk_ & 3));                        \
  }
#define DSM_Q80_COMMIT(K0)                                                                          \
  _Pragma("clang loop unroll(full)") for (int u = 0; u < 8; u++) {                                                   \
    const int c_ = 4 * u + p;                                                                       \
    *(u32x4*)&sA[r][c_ ^ (r & 15)] = av[u];                                                         \
    const int b0_ = slot_block((K0), u), b_ = b0_ < 0 ? 0 : b0_;                                    \
    const uint8_t* blk_ = wrow + (size_t)b_ * Q8_0_BYTES;                                           \
    const uint32_t sh_ = (uint32_t)((uintptr_t)(blk_ + 2 + 8 * p) & 3);                             \
    const uint32_t c0_ = sh_ ? __builtin_amdgcn_alignbyte(bc[u].y, bc[u].x, sh_) : bc[u].y;         \
    const uint32_t c1_ = sh_ ? __builtin_amdgcn_alignbyte(bc[u].z, bc[u].y, sh_) : bc[u].z;         \
    uint32_t o0_, o1_, o2_, o3_;                                                                    \
    i8x4_to_f16(c0_, o0_, o1_);                                                                     \
    i8x4_to_f16(c1_, o2_, o3_);                                                                     \
    sB[c_][r] = make_uint4(o0_, o1_, o2_, o3_);                                                     \
  }                                                                                                 \
  _Pragma("clang loop unroll(full)") for (int h = 0; h < 2; h++) {                                  \
    const int u = p + 4 * h;                                                                        \
    const int b0_ = slot_block((K0), u), b_ = b0_ < 0 ? 0 : b0_;                                    \
    const uint8_t* blk_ = wrow + (size_t)b_ * Q8_0_BYTES;                                           \
    const uint16_t db_ = ((uintptr_t)blk_ & 3) ? (uint16_t)(bd[h] >> 16) : (uint16_t)(bd[h] & 0xFFFF); \
    s_sw[r][u] = f16_to_f32_ftz(db_);                                                               \
    s_xs[u][r] = axs[h];                                                                            \
  }

  const int mt = w & 1, nt = w >> 1, hh = lane >> 5;
  const int arow_l = mt * 32 + (lane & 31), brow = nt * 32 + (lane & 31);
  float16v run, lv0, lv1, lv2, lv3, lv4;
  for (int i = 0; i < 16; i++) { run[i] = 0.0f; lv0[i] = lv1[i] = lv2[i] = lv3[i] = lv4[i] = 0.0f; }
  auto addv = [](const float16v& q, float16v& x) {
    for (int i = 0; i < 16; i++) x[i] = q[i] + x[i];
  };
  // fold class position k into the halving tree (a binary counter over k)
  auto fold = [&](int k) {
    float16v x = run;
    if (k & 1) {
      addv(lv0, x);
      if (k & 2) {
        addv(lv1, x);
        if (k & 4) {
          addv(lv2, x);
          if (k & 8) {
            addv(lv3, x);
            if (k & 16) { addv(lv4, x); lv0 = x; }  // k = 31: the row sum, kept in lv0
            else lv4 = x;
          } else lv3 = x;
        } else lv2 = x;
      } else lv1 = x;
    } else lv0 = x;
    for (int i = 0; i < 16; i++) run[i] = 0.0f;
  };

  DSM_Q80_ISSUE(kb)
  for (int k0 = kb; k0 < ke; k0 += G) {
    __syncthreads();
    DSM_Q80_COMMIT(k0)
    // past the end: re-read the first stage (unused); unconditional loads keep the wait counts exact
    DSM_Q80_ISSUE(k0 + G < ke ? k0 + G : kb)
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 8; u++) {
      if (u >= G * jmax) break;
      const int k = k0 + u / jmax, j = u % jmax;
      if (j < nblk(bitrev5(k))) {
        float16v acc;
        for (int i = 0; i < 16; i++) acc[i] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
          const int c = 4 * u + 2 * ks + hh;
          const half8 av8 = *(const half8*)&sA[arow_l][c ^ (arow_l & 15)];
          const half8 bv8 = *(const half8*)&sB[c][brow];
          acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(av8, bv8, acc, 0, 0, 0);
        }
        const float sw = s_sw[brow][u];
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const int m = mt * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
          run[i] = run[i] + (sw * s_xs[u][m]) * acc[i];
        }
      }
      if (j == jmax - 1) fold(k - kb);
    }
  }

#undef DSM_Q80_ISSUE
#undef DSM_Q80_COMMIT
  if (S > 1) {
    // the subtree of this workgroup's 32 / S classes: lv[log2(32 / S)]
    const float16v& sub = S == 2 ? lv4 : S == 4 ? lv3 : S == 8 ? lv2 : lv1;
    const int cols = kSwiglu ? 2 * a.out_dim : a.out_dim;
    const int col = kSwiglu ? nt * a.out_dim + n0 + (lane & 31) : n0 + nt * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int m = m0 + mt * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
      if (m < T) a.part[((size_t)split * T + m) * cols + col] = sub[i];
    }
    return;
  }
  if (!kSwiglu) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int m = m0 + mt * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
      if (m < T) a.out[(size_t)m * a.out_dim + n0 + nt * 32 + (lane & 31)] = lv0[i];
    }
    return;
  }
  __syncthreads();
  float* s_up = (float*)&sA[0][0];  // [64 tokens][32 rows]
  if (nt == 1) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int m = mt * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
      s_up[m * 32 + (lane & 31)] = lv0[i];
    }
  }
  __syncthreads();
  if (nt == 0) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int m = mt * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
      if (m0 + m >= T) continue;
      const float g = clamp_gate(lv0[i], a.clamp), u = clamp_up(s_up[m * 32 + (lane & 31)], a.clamp);
      a.out[(size_t)(m0 + m) * a.out_dim + n0 + (lane & 31)] = (g / (1.0f + expf_dsm(-g))) * u * 1.0f;
    }
  }
}

// One kernel per class length: kJ = 7 (in_dim 7168, the shared gate/up) and
// kJ = 2 (in_dim 1025 .. 2048, the shared down) as compile-time constants,
// any other length at run time (the unsuffixed kernels).
#define DSM_Q80_KERNEL(NAME, SW, J)                                                  \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) \
  void NAME(const Q80GemmArgs a) {                                                    \
    __shared__ Q80Smem sm;                                                            \
    q80_gemm<SW, J>(a, sm);                                                           \
  }
DSM_Q80_KERNEL(dsmoe_q80_gemm_swiglu, true, 0)
DSM_Q80_KERNEL(dsmoe_q80_gemm, false, 0)
DSM_Q80_KERNEL(dsmoe_q80_gemm_swiglu_j7, true, 7)
DSM_Q80_KERNEL(dsmoe_q80_gemm_j7, false, 7)
DSM_Q80_KERNEL(dsmoe_q80_gemm_swiglu_j2, true, 2)
DSM_Q80_KERNEL(dsmoe_q80_gemm_j2, false, 2)
#undef DSM_Q80_KERNEL

// ---------------------------------------------------------------------------
// Router logits for batches (matmul_f16, matmul.rs:57-105): workgroup =
// 8 experts x 16 tokens.  For each (token, expert) thread tx sums elements
// tx, tx+256, ... in order (f32 multiply, then add), and the halving tree
// 128 .. 1 over the 256 partials combines them, as in the per-row role of
// dsmoe_prep; each weight element loaded (and converted from f16, the
// larger part of the non-product work) serves 16 tokens and each activation
// element 8 experts.
// grid = ceil(E / 8) * ceil(T / 16), 256 threads.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void dsmoe_router_tile(const RouterLogitsArgs a) {
  constexpr int NE = 8, NT = 16;
  __shared__ float part[NE * 8][256];  // [expert * 8 + token][tx], eight tokens at a time
  const int neg = (a.E + NE - 1) / NE;
  const int e0 = (blockIdx.x % neg) * NE, t0 = (blockIdx.x / neg) * NT;
  const int tx = threadIdx.x, d = a.d, nb = d >> 8;
  // rows past E or T re-read the last valid one (never stored).  Loads are
  // raw buffer loads: the tensor's descriptor, the thread's constant byte
  // offset of (row, tx) and the element step as the scalar offset.
  uint32_t wo[NE], xo[NT];
#pragma unroll
  for (int k = 0; k < NE; k++) wo[k] = 2u * ((uint32_t)min(e0 + k, a.E - 1) * (uint32_t)d + (uint32_t)tx);
#pragma unroll
  for (int k = 0; k < NT; k++) xo[k] = 4u * ((uint32_t)min(t0 + k, a.T - 1) * (uint32_t)d + (uint32_t)tx);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, 2 * a.E * d, kBufDword3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, 4 * a.T * d, kBufDword3);
  float acc[NE][NT];
#pragma unroll
  for (int e = 0; e < NE; e++)
#pragma unroll
    for (int t = 0; t < NT; t++) acc[e][t] = 0.0f;
  // element j of this thread's slot: the next one's loads are issued before
  // the current one's products (a load past the end re-reads element 0 and is
  // never used)
  uint16_t wh[2][NE];
  float xv[2][NT];
  auto load = [&](int buf, int j) {
    const int jj = j < nb ? j : 0;
#pragma unroll
    for (int k = 0; k < NE; k++) wh[buf][k] = __builtin_amdgcn_raw_buffer_load_b16(rw, (int)wo[k], 512 * jj, 0);
#pragma unroll
    for (int k = 0; k < NT; k++)
      xv[buf][k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, (int)xo[k], 1024 * jj, 0));
  };
  auto products = [&](int buf) {
    float wv[NE];
#pragma unroll
    for (int k = 0; k < NE; k++) wv[k] = f16_to_f32_ftz_nb(wh[buf][k]);
#pragma unroll
    for (int e = 0; e < NE; e++)
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const float pr = wv[e] * xv[buf][t];
        acc[e][t] = acc[e][t] + pr;
      }
  };
  load(0, 0);
  for (int j = 0; j < nb; j += 2) {
    load(1, j + 1);
    products(0);
    if (j + 1 >= nb) break;
    load(0, j + 2);
    products(1);
  }
#pragma unroll
  for (int h = 0; h < NT / 8; h++) {
    if (h) __syncthreads();  // the previous half's tree is read out
#pragma unroll
    for (int e = 0; e < NE; e++)
#pragma unroll
      for (int t = 0; t < 8; t++) part[8 * e + t][tx] = acc[e][8 * h + t];
    __syncthreads();
    for (int s2 = 128, lg = 7; s2 > 0; s2 >>= 1, lg--) {
      for (int idx = tx; idx < 64 * s2; idx += 256) {
        const int pr = idx >> lg, i = idx & (s2 - 1);
        part[pr][i] += part[pr][i + s2];
      }
      __syncthreads();
    }
    if (tx < 64) {
      const int e = tx >> 3, t = 8 * h + (tx & 7);
      if (e0 + e < a.E && t0 + t < a.T) a.out[(size_t)(t0 + t) * a.E + e0 + e] = part[tx][0];
    }
  }
}


// ---------------------------------------------------------------------------
// Peak probes (no reference counterpart): the bench reports the sustained
// MFMA rate and HBM read rate of the box next to the published peaks.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void dsmoe_probe_mfma(const ProbeArgs a) {
  const int lane = threadIdx.x & 63;
  half8 x, y;
  for (int j = 0; j < 8; j++) {
    x[j] = (_Float16)(0.001f * (float)((lane + j) & 7));
    y[j] = (_Float16)(0.002f * (float)((lane * 3 + j) & 7));
  }
  float16v acc[8];
  for (int c = 0; c < 8; c++)
    for (int j = 0; j < 16; j++) acc[c][j] = 0.0f;
  for (int64_t it = 0; it < a.iters; it++) {
#pragma unroll
    for (int c = 0; c < 8; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x, y, acc[c], 0, 0, 0);
  }
  float s = 0.0f;
  for (int c = 0; c < 8; c++)
    for (int j = 0; j < 16; j++) s = s + acc[c][j];
  if (s == 1234.5f) a.sink[blockIdx.x] = s;  // never true; keeps the chain live
}

extern "C" __global__ __launch_bounds__(256) void dsmoe_probe_read(const ProbeArgs a) {
  uint32_t x = 0;
#pragma unroll 8
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n16; i += (uint64_t)gridDim.x * blockDim.x) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)a.src + i);
    x ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (x == 0x9E3779B9u) a.sink[blockIdx.x] = (float)x;  // data-dependent, almost never taken
}

// Finishes a split Q8_0 GEMM: the partial sums of the ksplit class groups
// added pairwise in split order (for ksplit = 2^s the groups are the subtrees
// of the halving tree's top s levels, in tree order), then SwiGLU (weight 1)
// when the GEMM had gate and up.  One thread per output.
extern "C" __global__ __launch_bounds__(256) void dsmoe_q80_combine(const Q80CombineArgs a) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)a.T * a.out_dim) return;
  const size_t t = i / a.out_dim, c = i % a.out_dim;
  const int cols = a.two ? 2 * a.out_dim : a.out_dim;
  const size_t plane = (size_t)a.T * cols;
  auto tree = [&](size_t col) {
    float v[8];
    for (int s = 0; s < a.ksplit; s++) v[s] = a.part[s * plane + t * cols + col];
    for (int w = a.ksplit; w > 1; w >>= 1)
      for (int s = 0; s < w / 2; s++) v[s] = v[2 * s] + v[2 * s + 1];
    return v[0];
  };
  const float g0 = tree(c);
  if (!a.two) { a.out[i] = g0; return; }
  const float g = clamp_gate(g0, a.clamp), u = clamp_up(tree(a.out_dim + c), a.clamp);
  a.out[i] = (g / (1.0f + expf_dsm(-g))) * u * 1.0f;
}
