// Host side of the dsmoe C ABI (include/dsmoe.h): argument validation,
// kernel code-object loading through hipModule, launch shapes, the
// per-layer launch sequence and the context's scratch buffers.
//
// The launch sequence of dsmoe_forward follows
// Session::decode_attn_out_and_ffn (engine/src/session.rs:1894-2155):
// shared expert (g) then router + routed experts (h).
#include "dsmoe.h"

#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>

#include "dsmoe_formats.h"
#include "dsmoe_kargs.h"
#include "dsmoe_synth.h"

using namespace dsm;

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

#define DSM_CHECK_HIP(expr)                                                              \
  do {                                                                                   \
    hipError_t _e = (expr);                                                              \
    if (_e != hipSuccess)                                                                \
      return fail(DSMOE_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(_e));     \
  } while (0)

#define DSM_TRY(expr)            \
  do {                           \
    int _rc = (expr);            \
    if (_rc != DSMOE_OK) return _rc; \
  } while (0)

// --------------------------------------------------------------------------
// IQ2_XXS level-tuple map used by the synthetic encoder: for each of the
// 3^8 tuples of magnitude levels {8, 25, 43}, the codebook entry with the
// smallest squared error (lowest index on ties).
// --------------------------------------------------------------------------
const std::vector<uint8_t>& lvlmap_host() {
  static std::vector<uint8_t> map;
  static std::once_flag once;
  std::call_once(once, [] {
    const int lv[3] = {8, 25, 43};
    map.resize(6561);
    for (int t = 0; t < 6561; t++) {
      int want[8], r = t;
      for (int i = 0; i < 8; i++) { want[i] = lv[r % 3]; r /= 3; }
      int best = 0;
      long best_err = -1;
      for (int g = 0; g < 256; g++) {
        long err = 0;
        for (int i = 0; i < 8; i++) {
          const int gb = (int)((kIq2xxsGrid[g] >> (8 * i)) & 0xFF);
          err += (long)(gb - want[i]) * (gb - want[i]);
        }
        if (best_err < 0 || err < best_err) { best_err = err; best = g; }
      }
      map[t] = (uint8_t)best;
    }
  });
  return map;
}

// --------------------------------------------------------------------------
// Code object + kernels, one set per device.
// --------------------------------------------------------------------------
enum Kern { K_PREP, K_ROUTER_SELECT, K_UP, K_MIDQ, K_DN, K_SWIGLU, K_MOE_SUM, K_DISPATCH, K_SYNTH,
            K_GU_GROUPED, K_DN_GROUPED, K_Q80_GEMM_SWIGLU, K_Q80_GEMM,
            K_ROUTER_TILE, K_UP_ROWS, K_DN_ROWS, K_Q80_GEMM_SWIGLU_J7, K_Q80_GEMM_J7, K_Q80_GEMM_SWIGLU_J2,
            K_Q80_GEMM_J2, K_HC_EXPAND, K_PROBE_MFMA, K_PROBE_READ, K_UP_EM, K_DN_EM, K_Q80_COMBINE, K_SELECT_HASH, K_RMS_NORM, K_HC_SPLIT_NORM,
            K_Q80_UNPACK, K_Q80_WIDE, K_Q80_WIDE_SW, K_ROUTER_TILE_S, K_COUNT };
const char* kKernNames[K_COUNT] = {"dsmoe_prep", "dsmoe_router_select", "dsmoe_up", "dsmoe_midq", "dsmoe_dn",
                                   "dsmoe_swiglu", "dsmoe_moe_sum", "dsmoe_dispatch", "dsmoe_synth",
                                   "dsmoe_gu_grouped", "dsmoe_dn_grouped", "dsmoe_q80_gemm_swiglu", "dsmoe_q80_gemm",
                                   "dsmoe_router_tile",
                                   "dsmoe_up_rows", "dsmoe_dn_rows", "dsmoe_q80_gemm_swiglu_j7", "dsmoe_q80_gemm_j7",
                                   "dsmoe_q80_gemm_swiglu_j2", "dsmoe_q80_gemm_j2", "dsmoe_hc_expand",
                                   "dsmoe_probe_mfma", "dsmoe_probe_read", "dsmoe_up_em", "dsmoe_dn_em",
                                   "dsmoe_q80_combine", "dsmoe_router_select_hash",
                                   "dsmoe_rms_norm_plain", "dsmoe_hc_split_norm", "dsmoe_q80_unpack", "dsmoe_q80_wide",
                                   "dsmoe_q80_wide_swiglu", "dsmoe_router_tile_s"};
// code object of each kernel: 0 = dsmoe_kernels.hsaco, 1 = dsmoe_gemm.hsaco (same directory)
const int kKernModule[K_COUNT] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 0, 0, 1, 1, 1, 1, 0, 1, 1, 0, 0, 1, 0, 0, 0,
                                  1, 1, 1, 1};
static_assert(DSMOE_GROUPED_TILE_M == kGuBM, "header and kernels disagree on the grouped tile");

extern "C" int dsmoe_noalloc_setup(void** ptr, size_t* bytes);  // dsmoe_noalloc.hip

struct DeviceState {
  bool loaded = false;
  hipModule_t mod = nullptr;
  hipModule_t mod_gemm = nullptr;
  hipFunction_t fn[K_COUNT] = {};
  uint8_t* d_lvlmap = nullptr;
  uint8_t* noalloc = nullptr;  // this device's static scratch (dsmoe_noalloc.hip)
  size_t noalloc_bytes = 0;
};

constexpr int kMaxDevices = 64;
DeviceState g_dev[kMaxDevices];
std::mutex g_mu;

std::string default_code_object() {
  Dl_info info;
  if (dladdr((void*)&dsmoe_version, &info) && info.dli_fname) {
    std::string p(info.dli_fname);
    const size_t slash = p.rfind('/');
    return (slash == std::string::npos ? std::string(".") : p.substr(0, slash)) + "/dsmoe_kernels.hsaco";
  }
  return "dsmoe_kernels.hsaco";
}

int load_device(const char* path, DeviceState** out) {
  int dev = 0;
  DSM_CHECK_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(DSMOE_ERR_UNSUPPORTED, "device index out of range");
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState& st = g_dev[dev];
  if (!st.loaded) {
    const std::string p = path ? std::string(path) : default_code_object();
    hipError_t e = hipModuleLoad(&st.mod, p.c_str());
    if (e != hipSuccess)
      return fail(DSMOE_ERR_MODULE, "hipModuleLoad(" + p + "): " + hipGetErrorString(e));
    const size_t slash = p.rfind('/');
    const std::string pg = (slash == std::string::npos ? std::string(".") : p.substr(0, slash)) + "/dsmoe_gemm.hsaco";
    e = hipModuleLoad(&st.mod_gemm, pg.c_str());
    if (e != hipSuccess)
      return fail(DSMOE_ERR_MODULE, "hipModuleLoad(" + pg + "): " + hipGetErrorString(e));
    for (int k = 0; k < K_COUNT; k++) {
      e = hipModuleGetFunction(&st.fn[k], kKernModule[k] ? st.mod_gemm : st.mod, kKernNames[k]);
      if (e != hipSuccess)
        return fail(DSMOE_ERR_MODULE, std::string("hipModuleGetFunction(") + kKernNames[k] + "): " +
                                          hipGetErrorString(e));
    }
    void* sp = nullptr;
    size_t sb = 0;
    const int se = dsmoe_noalloc_setup(&sp, &sb);
    if (se != 0)
      return fail(DSMOE_ERR_HIP, std::string("static scratch set-up: ") + hipGetErrorString((hipError_t)se));
    st.noalloc = (uint8_t*)sp;
    st.noalloc_bytes = sb;
    st.loaded = true;
  }
  *out = &st;
  return DSMOE_OK;
}

template <class A>
int launch(Kern k, dim3 grid, dim3 block, size_t shmem, dsmoe_stream_t stream, const A& args) {
  DeviceState* st = nullptr;
  DSM_TRY(load_device(nullptr, &st));
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return DSMOE_OK;
  if (shmem > 160 * 1024) return fail(DSMOE_ERR_UNSUPPORTED, "LDS request above 160 KiB");
  A copy = args;
  void* params[] = {(void*)&copy};
  DSM_CHECK_HIP(hipModuleLaunchKernel(st->fn[k], grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                      (unsigned)shmem, (hipStream_t)stream, params, nullptr));
  return DSMOE_OK;
}

inline int align_up(int v, int a) { return (v + a - 1) / a * a; }
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Launch shapes.  Each matvec role streams one work item (a weight block or
// block pair) per thread; R rows per workgroup are chosen so the items fit
// the workgroup (<= 1024 threads) and the grid has at least ~2 workgroups
// per CU (256 CUs).
constexpr int kMinWgs = 512;
constexpr int kDecodeMaxT = kMaxDecodeT;  // row-streaming (matvec) launches up to 8 tokens, batch paths above
constexpr int kEmMaxLoad = 4;    // pairs per expert (on average) up to which batches run expert-major
constexpr int kEmDnMaxLoad = 2;  // ... and up to which the down does too (above: the int8 grouped down)
constexpr int kQ80MaxSplit = 8;  // class groups of a split shared-expert GEMM (up to 256 tokens)
// Pairs per expert-major chunk: a chunk keeps its activations in LDS, so a
// smaller chunk leaves room for more workgroups per compute unit, a larger
// one streams a busy expert's rows fewer times.  4 measured best on c3
// (T = 32, about 1.5 pairs per used expert) and c4 (T = 128, about 4)
// against 1, 2 and 8.
int em_pairs() { return 4; }

int pow2_floor(int v) {
  int p = 1;
  while (p * 2 <= v) p *= 2;
  return p;
}

struct Shape {
  int R;       // rows per workgroup
  int block;   // threads per workgroup
  int tiles;   // workgroups along the rows
};

// items_per_row: work items per output row; epi_per_row: epilogue threads
// per output row; rows: output rows; work: the grid's second extent.
Shape matvec_shape(int items_per_row, int epi_per_row, int rows, int work, int max_block = 1024) {
  const int per = std::max(items_per_row, epi_per_row);
  int R = std::max(1, std::min(64, pow2_floor(std::max(1, max_block / std::max(1, per)))));
  while (R > 1 && (long)((rows + R - 1) / R) * work < kMinWgs) R /= 2;
  const int block = std::min(1024, align_up(std::max(64, R * per), 64));
  return {R, block, (rows + R - 1) / R};
}

// Row-streaming launches (dsmoe_up_rows / dsmoe_dn_rows): shapes they take and
// their LDS.  Everything else runs the per-item launches (dsmoe_up / dsmoe_dn).
bool up_rows_fits(int d) { return d % 512 == 0 && d <= 8192; }
bool dn_rows_fits(int I, int k) { return k <= 8 && I % 256 == 0 && I <= 2048; }
bool q80_rows_fits(int in_dim) { return in_dim % 64 == 0 && in_dim <= 8192; }
constexpr int kUpRowsR = 32, kDnRowsR = 8;
size_t gate_up_rows_lds(int nb) { return 3072 + (size_t)align_up(nb, 4) * 4 + (size_t)nb * 272 + 256; }
size_t q80_rows_lds(int nb) { return (size_t)align_up(nb, 4) * 4 + (size_t)nb * 32 + 32; }
// Experts per lane of the one-wave selection (E = 64 * P, groups of whole
// lane blocks of 1..16 lanes), or 0 when the selection needs the LDS form.
// Expert-major launches (dsmoe_up_em / dsmoe_dn_em): shapes they take.  The
// gate/up workgroup stages up to kEmPairs activations in LDS (at most 64 KB).
size_t gate_up_em_lds(int nb, int np = kEmPairs) { return 3072 + (size_t)np * nb * 272; }
size_t down_em_lds(int nb, int np = kEmPairs) { return (size_t)np * nb * 304; }
bool em_fits(const dsmoe_config& cf) {
  return up_rows_fits(cf.d_model) && gate_up_em_lds(cf.d_model / 256) <= 64 * 1024 && cf.d_ff <= 2048 &&
         cf.d_ff % 256 == 0;
}
int q80_rows_tiles(int out_dim, bool two) { return two ? (out_dim + 3) / 4 : (out_dim + 7) / 8; }
size_t gate_up_lds(int nb, int R) { return 3072 + (size_t)align_up(nb, 4) * 4 + (size_t)nb * 272 + (size_t)2 * R * nb * 4; }
size_t down_lds(int K, int nb, int R) {
  return (size_t)align_up(K * nb, 4) * 4 + (size_t)K * nb * 32 + (size_t)K * nb * 272 + (size_t)K * R * nb * 4 +
         (size_t)K * R * 4;
}
size_t q80_lds(int nb, int nmat, int R) { return (size_t)align_up(nb, 4) * 4 + (size_t)nb * 32 + (size_t)nmat * R * nb * 4; }
size_t select_lds(int E) { return (size_t)E * 20 + 128 * 4 + 64 * 4 + 32 * 8; }
size_t router_lds(int) { return 8 * 256 * 4; }

int validate_cfg(const dsmoe_config* c) {
  if (!c) return fail(DSMOE_ERR_INVALID, "config is NULL");
  if (c->d_model <= 0 || c->d_model % 512 || c->d_model > 8192)
    return fail(DSMOE_ERR_UNSUPPORTED, "d_model must be a positive multiple of 512, at most 8192");
  if (c->d_ff <= 0 || c->d_ff % 256) return fail(DSMOE_ERR_INVALID, "d_ff must be a positive multiple of 256");
  if (c->n_expert < 1 || c->n_expert > 1024) return fail(DSMOE_ERR_UNSUPPORTED, "n_expert must be in 1..1024");
  if (c->top_k < 1 || c->top_k > 32 || c->top_k > c->n_expert)
    return fail(DSMOE_ERR_INVALID, "top_k must be in 1..min(32, n_expert)");
  if (c->n_group < 1) return fail(DSMOE_ERR_INVALID, "n_group must be >= 1");
  if (c->n_group > 1) {
    if (c->n_group > 64 || c->n_expert % c->n_group)
      return fail(DSMOE_ERR_INVALID, "n_group must divide n_expert and be <= 64");
    if (c->topk_group < 1 || c->topk_group > c->n_group)
      return fail(DSMOE_ERR_INVALID, "topk_group must be in 1..n_group");
    if (c->top_k > c->topk_group * (c->n_expert / c->n_group))
      return fail(DSMOE_ERR_INVALID, "top_k exceeds the experts of the kept groups");
  }
  if (!(c->route_scale == c->route_scale)) return fail(DSMOE_ERR_INVALID, "route_scale is NaN");
  if (c->shared_fmt < -1 || c->shared_fmt > 1) return fail(DSMOE_ERR_INVALID, "shared_fmt must be -1, 0 or 1");
  if (c->shared_fmt == 0 && (c->d_ff_shared <= 0 || c->d_ff_shared % 64))
    return fail(DSMOE_ERR_UNSUPPORTED, "Q8_0 shared expert needs d_ff_shared a positive multiple of 64");
  if (c->shared_fmt == 1 && (c->d_ff_shared <= 0 || c->d_ff_shared % 256))
    return fail(DSMOE_ERR_INVALID, "IQ2_XXS/Q2_K shared expert needs d_ff_shared a multiple of 256");
  return DSMOE_OK;
}

}  // namespace

namespace dsm_gguf {
// The GGUF reader (dsmoe_gguf.cpp) reports through the same last-error slot.
int fail(int code, const std::string& msg) { return ::fail(code, msg); }
}  // namespace dsm_gguf

// ==========================================================================
// C ABI
// ==========================================================================
extern "C" {

const char* dsmoe_version(void) { return "dsmoe 0.2 (gfx950)"; }
const char* dsmoe_last_error(void) { return g_err.c_str(); }

int dsmoe_init(const char* code_object_path) {
  DeviceState* st = nullptr;
  return load_device(code_object_path, &st);
}

// Batches of more than 8 tokens take the router logits from dsmoe_router_tile
// (8 experts x 8 tokens per workgroup, same float order); the prep launch
// keeps the quantizations.
static constexpr int kRouterTileMinT = 9;

// Workgroups of the quantization roles of dsmoe_prep / dsmoe_midq: four Q8_K
// blocks (one per wave) or 32 Q8_0 blocks where the wave forms apply, else
// one Q8_K block / 8 Q8_0 blocks of one row.
static int q8k_units(const Q8KArgs& q) {
  return q8k_waves_ok(q) ? ((q.in_dim / 256) * q.rows + 3) / 4 : (q.in_dim / 256) * q.rows;
}
static int q80_units(const Q80Args& q) {
  if (q80_waves_ok(q)) return ((q.in_dim / 32) * q.rows + 31) / 32;
  return ((q.in_dim + 31) / 32 + 7) / 8 * q.rows;
}

static int midq_impl(const Q8KArgs* qa, const Q8KArgs* qb, const Q80Args* q80, dsmoe_stream_t stream);

static int prep_impl(const RouterLogitsArgs* r, const Q8KArgs* q8k, const Q80Args* q80, dsmoe_stream_t stream) {
  // the batch kernel addresses x and the router with 32-bit buffer offsets
  if (r && r->T >= kRouterTileMinT && (int64_t)r->T * r->d * 4 < ((int64_t)1 << 31) &&
      (int64_t)r->E * r->d * 2 < ((int64_t)1 << 31)) {
    // 8 x 12 tiles unless their grid would leave most compute units idle:
    // below 128 of them (c3, T = 32: 96) the 4 x 8 tiles measured ~1 % faster
    // per layer, at c4 (T = 128, where the concurrent shared expert is the
    // longer chain) ~0.6 % slower
    const unsigned big = (unsigned)(((r->E + 7) / 8) * ((r->T + 11) / 12));
    if (big < 128u)
      DSM_TRY(launch(K_ROUTER_TILE_S, dim3(((r->E + 3) / 4) * ((r->T + 7) / 8)), dim3(256), 0, stream, *r));
    else
      DSM_TRY(launch(K_ROUTER_TILE, dim3(big), dim3(256), 0, stream, *r));
    r = nullptr;
    if (!q8k && !q80) return DSMOE_OK;
  }
  // without router rows the quantizations run in dsmoe_midq (same roles; its
  // registers allow more waves than dsmoe_prep's router rows need)
  if (!r) return midq_impl(q8k, nullptr, q80, stream);
  PrepArgs a{};
  if (r) { a.router = *r; a.n_router = r->E * ((r->T + 7) / 8); }
  if (q8k) { a.q8k = *q8k; a.n_q8k = q8k_units(*q8k); }
  if (q80) { a.q80 = *q80; a.n_q80 = q80_units(*q80); }
  const size_t lds = std::max<size_t>(r ? router_lds(r->d) : 0, 2 * 256 * 4 + 256);
  return launch(K_PREP, dim3(a.n_router + a.n_q8k + a.n_q80), dim3(256), lds, stream, a);
}

int dsmoe_router_logits(const uint16_t* w, const float* x, float* out, int32_t d, int32_t E, int32_t T,
                        dsmoe_stream_t stream) {
  if (!w || !x || !out) return fail(DSMOE_ERR_INVALID, "router_logits: null pointer");
  if (d <= 0 || d % 256 || E <= 0 || T < 0) return fail(DSMOE_ERR_INVALID, "router_logits: d must be a multiple of 256");
  if (d > 65536) return fail(DSMOE_ERR_UNSUPPORTED, "router_logits: d must be <= 65536");
  RouterLogitsArgs a{w, x, out, d, E, T};
  return prep_impl(&a, nullptr, nullptr, stream);
}

int dsmoe_router_select(const dsmoe_config* cfg, const float* logits, const float* bias, int32_t T,
                        float* probs, int32_t* selected, float* weights, dsmoe_stream_t stream) {
  if (!cfg) return fail(DSMOE_ERR_INVALID, "router_select: config is NULL");
  if (!logits || !selected || !weights) return fail(DSMOE_ERR_INVALID, "router_select: null pointer");
  if (cfg->has_bias && !bias) return fail(DSMOE_ERR_INVALID, "router_select: has_bias without bias");
  if (cfg->n_expert < 1 || cfg->n_expert > 1024) return fail(DSMOE_ERR_UNSUPPORTED, "router_select: n_expert in 1..1024");
  if (cfg->top_k < 1 || cfg->top_k > 32 || cfg->top_k > cfg->n_expert) return fail(DSMOE_ERR_INVALID, "router_select: bad top_k");
  if (cfg->n_group > 1 && (cfg->n_group > 64 || cfg->n_expert % cfg->n_group || cfg->topk_group < 1 ||
                           cfg->topk_group > cfg->n_group))
    return fail(DSMOE_ERR_INVALID, "router_select: bad grouping");
  if (T < 0) return fail(DSMOE_ERR_INVALID, "router_select: T < 0");
  RouterSelectArgs a{logits, cfg->has_bias ? bias : nullptr, probs, selected, weights, T, cfg->n_expert,
                     cfg->top_k, cfg->n_group > 1 ? cfg->n_group : 1, cfg->topk_group, cfg->has_bias ? 1 : 0,
                     cfg->route_scale};
  return launch(K_ROUTER_SELECT, dim3(T), dim3(256), select_lds(cfg->n_expert), stream, a);
}

int dsmoe_router_select_hash(const dsmoe_config* cfg, const float* logits, const int32_t* hash, int32_t hash_rows,
                             const int32_t* tokens, int32_t token_scalar, int32_t T, float* probs, int32_t* selected,
                             float* weights, dsmoe_stream_t stream) {
  if (!cfg || !logits || !hash || !selected || !weights) return fail(DSMOE_ERR_INVALID, "router_select_hash: null pointer");
  if (T < 0 || hash_rows < 1 || cfg->n_expert < 1 || cfg->top_k < 1)
    return fail(DSMOE_ERR_INVALID, "router_select_hash: bad shape");
  HashSelectArgs a{logits, hash, tokens, probs, selected, weights, token_scalar, hash_rows, T, cfg->n_expert,
                   cfg->top_k, cfg->route_scale};
  return launch(K_SELECT_HASH, dim3(T), dim3(256), 0, stream, a);
}

static int midq_impl(const Q8KArgs* qa, const Q8KArgs* qb, const Q80Args* q80, dsmoe_stream_t stream) {
  MidqArgs a{};
  if (qa) { a.q8k_a = *qa; a.n_a = q8k_units(*qa); }
  if (qb) { a.q8k_b = *qb; a.n_b = q8k_units(*qb); }
  if (q80) { a.q80 = *q80; a.n_q80 = q80_units(*q80); }
  return launch(K_MIDQ, dim3(a.n_a + a.n_b + a.n_q80), dim3(256), 0, stream, a);
}

int dsmoe_q8k_quantize(const float* x, void* out, int32_t in_dim, int32_t rows, dsmoe_stream_t stream) {
  if (!x || !out) return fail(DSMOE_ERR_INVALID, "q8k_quantize: null pointer");
  if (in_dim <= 0 || in_dim % 256 || rows < 0) return fail(DSMOE_ERR_INVALID, "q8k_quantize: in_dim must be a multiple of 256");
  Q8KArgs a{x, (uint8_t*)out, in_dim, rows};
  return midq_impl(&a, nullptr, nullptr, stream);
}

int dsmoe_q8k_quantize_h(const float* x, void* out, uint16_t* out_h, int32_t in_dim, int32_t rows,
                         dsmoe_stream_t stream) {
  if (!x || !out || !out_h) return fail(DSMOE_ERR_INVALID, "q8k_quantize_h: null pointer");
  if (in_dim <= 0 || in_dim % 256 || rows < 0)
    return fail(DSMOE_ERR_INVALID, "q8k_quantize_h: in_dim must be a multiple of 256");
  Q8KArgs a{x, (uint8_t*)out, in_dim, rows, out_h};
  return midq_impl(&a, nullptr, nullptr, stream);
}

int dsmoe_q8k_quantize_i8(const float* x, void* out, int8_t* out_i8, uint16_t* bsum_h, int32_t in_dim, int32_t rows,
                          dsmoe_stream_t stream) {
  if (!x || !out || !out_i8 || !bsum_h) return fail(DSMOE_ERR_INVALID, "q8k_quantize_i8: null pointer");
  if (in_dim <= 0 || in_dim % 256 || rows < 0)
    return fail(DSMOE_ERR_INVALID, "q8k_quantize_i8: in_dim must be a multiple of 256");
  if (!aligned16(out_i8)) return fail(DSMOE_ERR_INVALID, "q8k_quantize_i8: out_i8 must be 16-byte aligned");
  Q8KArgs a{x, (uint8_t*)out, in_dim, rows, nullptr, out_i8, bsum_h};
  return midq_impl(&a, nullptr, nullptr, stream);
}

int dsmoe_q8_0_quantize_h(const float* x, int8_t* xq, float* xscale, uint16_t* out_h, int32_t in_dim, int32_t rows,
                          dsmoe_stream_t stream) {
  if (!x || !xq || !xscale || !out_h) return fail(DSMOE_ERR_INVALID, "q8_0_quantize_h: null pointer");
  if (in_dim <= 0 || rows < 0) return fail(DSMOE_ERR_INVALID, "q8_0_quantize_h: bad shape");
  Q80Args a{x, xq, xscale, in_dim, rows, out_h};
  return midq_impl(nullptr, nullptr, &a, stream);
}

int dsmoe_q8_0_quantize(const float* x, int8_t* xq, float* xscale, int32_t in_dim, int32_t rows,
                        dsmoe_stream_t stream) {
  if (!x || !xq || !xscale) return fail(DSMOE_ERR_INVALID, "q8_0_quantize: null pointer");
  if (in_dim <= 0 || rows < 0) return fail(DSMOE_ERR_INVALID, "q8_0_quantize: bad shape");
  Q80Args a{x, xq, xscale, in_dim, rows};
  return midq_impl(nullptr, nullptr, &a, stream);
}

// Shapes + argument blocks of the matvec roles (validated by the callers).
static GateUpArgs gate_up_args(const void* gate, const void* up, const void* xq, const int32_t* selected,
                               const float* weights, const uint32_t* pair_list, float* gate_out, float* up_out,
                               float* mid_out, int d, int I, int k, int E, float clamp, int n_work, Shape* sh,
                               int max_block = 512) {
  const int nbp = d / 512;
  *sh = matvec_shape(2 * nbp, 16, I, n_work, max_block);
  return GateUpArgs{(const uint8_t*)gate, (const uint8_t*)up, (const uint8_t*)xq, selected, weights, pair_list,
                    gate_out, up_out, mid_out, d, I, k, sh->R, E, clamp};
}

static DownArgs down_args(const void* down, const void* midq, const int32_t* selected, float* down_out, float* out,
                          int d, int I, int k, int E, int T, Shape* sh, int max_block = 1024) {
  const int nb = I / 256;
  *sh = matvec_shape(k * nb, 8 * k, d, T, max_block);
  return DownArgs{(const uint8_t*)down, (const uint8_t*)midq, selected, out, down_out, d, I, k, sh->R, E};
}

static Q80MatvecArgs q80_args(const void* w0, const void* w1, const int8_t* xq, const float* xs, float* out0,
                              float* out1, float* mid, int in_dim, int out_dim, int T, float clamp, Shape* sh,
                              int max_block = 512) {
  const int nbp = in_dim / 64, nmat = w1 ? 2 : 1;
  *sh = matvec_shape(nmat * nbp, nmat * 32, out_dim, T, max_block);
  return Q80MatvecArgs{(const uint8_t*)w0, (const uint8_t*)w1, xq, xs, out0, out1, mid, in_dim, out_dim, sh->R, clamp};
}

static int check_gate_up(const void* gate, const void* up, const void* xq, const float* mid_out, int d, int I, int k) {
  if (!gate || !up || !xq || !mid_out) return fail(DSMOE_ERR_INVALID, "gate_up_mid: null pointer");
  if (!aligned16(gate) || !aligned16(up)) return fail(DSMOE_ERR_INVALID, "gate_up_mid: weights must be 16-byte aligned");
  if (d <= 0 || d % 512) return fail(DSMOE_ERR_UNSUPPORTED, "gate_up_mid: d must be a multiple of 512");
  if (I <= 0 || k <= 0) return fail(DSMOE_ERR_INVALID, "gate_up_mid: bad shape");
  if (gate_up_lds(d / 256, 1) > 64 * 1024) return fail(DSMOE_ERR_UNSUPPORTED, "gate_up_mid: d too large");
  return DSMOE_OK;
}

static int check_down(const void* down, const void* midq, int d, int I, int k) {
  if (!down || !midq) return fail(DSMOE_ERR_INVALID, "down: null pointer");
  if (!aligned16(down)) return fail(DSMOE_ERR_INVALID, "down: weights must be 16-byte aligned");
  if (d <= 0 || I <= 0 || I % 256 || k <= 0) return fail(DSMOE_ERR_INVALID, "down: bad shape");
  if (down_lds(k, I / 256, 1) > 64 * 1024) return fail(DSMOE_ERR_UNSUPPORTED, "down: k * I too large for one workgroup");
  return DSMOE_OK;
}

static int check_q80(const void* w0, const void* w1, const int8_t* xq, const float* xs, int in_dim, int out_dim) {
  if (!w0 || !xq || !xs) return fail(DSMOE_ERR_INVALID, "q8_0_matvec: null pointer");
  if (!aligned16(w0) || (w1 && !aligned16(w1))) return fail(DSMOE_ERR_INVALID, "q8_0_matvec: weights must be 16-byte aligned");
  if (in_dim <= 0 || in_dim % 64 || out_dim <= 0) return fail(DSMOE_ERR_UNSUPPORTED, "q8_0_matvec: in_dim must be a multiple of 64");
  if (q80_lds(in_dim / 32, 2, 1) > 64 * 1024) return fail(DSMOE_ERR_UNSUPPORTED, "q8_0_matvec: in_dim too large");
  return DSMOE_OK;
}

int dsmoe_gate_up_mid(const void* gate, const void* up, const void* xq, const int32_t* selected,
                      const float* weights, float* gate_out, float* up_out, float* mid_out, int32_t d,
                      int32_t I, int32_t T, int32_t k, int32_t E, float clamp, dsmoe_stream_t stream) {
  if (T < 0) return fail(DSMOE_ERR_INVALID, "gate_up_mid: T < 0");
  if (E < 1) return fail(DSMOE_ERR_INVALID, "gate_up_mid: E < 1");
  DSM_TRY(check_gate_up(gate, up, xq, mid_out, d, I, k));
  UpArgs a{};
  Shape sh;
  a.gu = gate_up_args(gate, up, xq, selected, weights, nullptr, gate_out, up_out, mid_out, d, I, k, E, clamp, T * k, &sh);
  a.gu_work = T * k;
  if (up_rows_fits(d)) {
    a.gu_tiles = (I + kUpRowsR - 1) / kUpRowsR;
    return launch(K_UP_ROWS, dim3(a.gu_tiles * a.gu_work), dim3(256), gate_up_rows_lds(d / 256), stream, a);
  }
  a.gu_tiles = sh.tiles;
  return launch(K_UP, dim3(a.gu_tiles * a.gu_work), dim3(sh.block), gate_up_lds(d / 256, sh.R), stream, a);
}

int dsmoe_down(const void* down, const void* midq, const int32_t* selected, float* down_out, float* out,
               int32_t d, int32_t I, int32_t T, int32_t k, int32_t E, dsmoe_stream_t stream) {
  if (!down_out && !out) return fail(DSMOE_ERR_INVALID, "down: null pointer");
  if (T < 0) return fail(DSMOE_ERR_INVALID, "down: bad shape");
  if (E < 1) return fail(DSMOE_ERR_INVALID, "down: E < 1");
  DSM_TRY(check_down(down, midq, d, I, k));
  DnArgs a{};
  Shape sh;
  a.dn = down_args(down, midq, selected, down_out, out, d, I, k, E, T, &sh);
  a.dn_work = T;
  if (dn_rows_fits(I, k)) {
    a.dn_tiles = (d + kDnRowsR - 1) / kDnRowsR;
    return launch(K_DN_ROWS, dim3(a.dn_tiles * a.dn_work), dim3(256), down_lds(k, I / 256, 0), stream, a);
  }
  a.dn_tiles = sh.tiles;
  return launch(K_DN, dim3(a.dn_tiles * a.dn_work), dim3(sh.block), down_lds(k, I / 256, sh.R), stream, a);
}

int dsmoe_moe_sum(const float* down, float* out, int32_t d, int32_t k, int32_t T, dsmoe_stream_t stream) {
  if (!down || !out) return fail(DSMOE_ERR_INVALID, "moe_sum: null pointer");
  if (d <= 0 || k <= 0 || T < 0) return fail(DSMOE_ERR_INVALID, "moe_sum: bad shape");
  MoeSumArgs a{down, out, d, k, T};
  const long n = moe_sum_vec_ok(a) ? (long)T * d / 4 : (long)T * d;  // threads
  return launch(K_MOE_SUM, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a);
}

int dsmoe_q8_0_matvec(const void* w, const int8_t* xq, const float* xscale, float* out, int32_t in_dim,
                      int32_t out_dim, int32_t T, dsmoe_stream_t stream) {
  if (!out) return fail(DSMOE_ERR_INVALID, "q8_0_matvec: null pointer");
  if (T < 0) return fail(DSMOE_ERR_INVALID, "q8_0_matvec: T < 0");
  DSM_TRY(check_q80(w, nullptr, xq, xscale, in_dim, out_dim));
  DnArgs a{};
  Shape sh;
  a.sh_q80 = q80_args(w, nullptr, xq, xscale, out, nullptr, nullptr, in_dim, out_dim, T, 0.0f, &sh);
  a.sh_work = T;
  a.sh_fmt = 0;
  if (q80_rows_fits(in_dim)) {
    a.sh_tiles = q80_rows_tiles(out_dim, false);
    return launch(K_DN_ROWS, dim3(a.sh_tiles * a.sh_work), dim3(256), q80_rows_lds(in_dim / 32), stream, a);
  }
  a.sh_tiles = sh.tiles;
  return launch(K_DN, dim3(a.sh_tiles * a.sh_work), dim3(sh.block), q80_lds(in_dim / 32, 1, sh.R), stream, a);
}

int dsmoe_probe(int32_t kind, const void* src, size_t bytes, int64_t iters, float* sink, dsmoe_stream_t stream) {
  if (!sink) return fail(DSMOE_ERR_INVALID, "probe: sink is NULL");
  int dev = 0, cus = 0;
  DSM_CHECK_HIP(hipGetDevice(&dev));
  DSM_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  if (kind == 0) {
    if (iters < 1) return fail(DSMOE_ERR_INVALID, "probe: iters < 1");
    ProbeArgs a{nullptr, sink, 0, iters};
    return launch(K_PROBE_MFMA, dim3(2u * cus), dim3(256), 0, stream, a);  // two waves per SIMD
  }
  if (kind == 1) {
    if (!src || bytes < 16 || ((uintptr_t)src & 15)) return fail(DSMOE_ERR_INVALID, "probe: bad source buffer");
    ProbeArgs a{(const uint4*)src, sink, bytes / 16, 0};
    return launch(K_PROBE_READ, dim3(8u * cus), dim3(256), 0, stream, a);
  }
  return fail(DSMOE_ERR_INVALID, "probe: unknown kind");
}

int dsmoe_rms_norm_plain(const float* x, float* out, int32_t n, int32_t rows, float eps, dsmoe_stream_t stream) {
  if (!x || !out) return fail(DSMOE_ERR_INVALID, "rms_norm_plain: null pointer");
  if (n < 1 || rows < 0) return fail(DSMOE_ERR_INVALID, "rms_norm_plain: bad shape");
  RmsNormArgs a{x, out, n, rows, eps};
  return launch(K_RMS_NORM, dim3(rows), dim3(256), 0, stream, a);
}

int dsmoe_hc_split_norm(const float* mix, const float* scale, const float* base, const float* residual_hc,
                        const float* norm_w, float* split, float* out, float* norm_out, int32_t n_embd, int32_t n_hc,
                        int32_t n_rows, int32_t sinkhorn_iters, float eps, float norm_eps, dsmoe_stream_t stream) {
  if (!mix || !scale || !base || !residual_hc || !norm_w || !split || !out || !norm_out)
    return fail(DSMOE_ERR_INVALID, "hc_split_norm: null pointer");
  if (n_hc != 4) return fail(DSMOE_ERR_UNSUPPORTED, "hc_split_norm: n_hc must be 4 (hc.rs:337)");
  if (n_embd < 1 || n_rows < 0 || sinkhorn_iters < 0) return fail(DSMOE_ERR_INVALID, "hc_split_norm: bad shape");
  HcSplitNormArgs a{mix, scale, base, residual_hc, norm_w, split, out, norm_out, n_embd, n_rows, sinkhorn_iters,
                    eps, norm_eps};
  return launch(K_HC_SPLIT_NORM, dim3(n_rows), dim3(256), 0, stream, a);
}

int dsmoe_hc_expand(const float* block_out, const float* block_add, const float* residual_hc, const float* split,
                    float* out_hc, int32_t n_embd, int32_t n_hc, int32_t n_tokens, int32_t mix_hc, int32_t has_add,
                    dsmoe_stream_t stream) {
  if (!block_out || !residual_hc || !split || !out_hc || (has_add && !block_add))
    return fail(DSMOE_ERR_INVALID, "hc_expand: null pointer");
  if (n_embd < 0 || n_hc < 1 || n_tokens < 0 || mix_hc < 2 * n_hc + n_hc * n_hc)
    return fail(DSMOE_ERR_INVALID, "hc_expand: bad shape (mix_hc must hold pre, post and comb)");
  HcExpandArgs a{block_out, has_add ? block_add : nullptr, residual_hc, split, out_hc, n_embd, n_hc, n_tokens, mix_hc,
                 has_add ? 1 : 0};
  const size_t n = (size_t)n_tokens * n_hc * n_embd;
  const size_t threads = hc_expand_vec_ok(a) ? n / 4 : n;
  if ((threads + 255) / 256 > 0x7FFFFFFF) return fail(DSMOE_ERR_UNSUPPORTED, "hc_expand: too large");
  return launch(K_HC_EXPAND, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, a);
}

int dsmoe_swiglu(const float* gate, const float* up, float* out, int32_t n, float clamp, float weight,
                 dsmoe_stream_t stream) {
  if (!gate || !up || !out) return fail(DSMOE_ERR_INVALID, "swiglu: null pointer");
  if (n < 0) return fail(DSMOE_ERR_INVALID, "swiglu: n < 0");
  SwigluArgs a{gate, up, out, n, clamp, weight};
  return launch(K_SWIGLU, dim3((n + 255) / 256), dim3(256), 0, stream, a);
}

int dsmoe_dispatch(const int32_t* selected, int32_t pairs, int32_t E, int32_t block_m, uint32_t* counts,
                   uint32_t* offsets, uint32_t* sorted_pairs, uint32_t* tile_offsets, uint32_t* tile_experts,
                   uint32_t* tile_starts, dsmoe_stream_t stream) {
  if (!selected || !counts || !offsets || !sorted_pairs) return fail(DSMOE_ERR_INVALID, "dispatch: null pointer");
  if (E < 1 || E > 512) return fail(DSMOE_ERR_UNSUPPORTED, "dispatch: E must be in 1..512");
  if (pairs < 0 || block_m < 1) return fail(DSMOE_ERR_INVALID, "dispatch: bad shape");
  if (tile_offsets && (!tile_experts || !tile_starts)) return fail(DSMOE_ERR_INVALID, "dispatch: partial tile outputs");
  DispatchArgs a{selected, counts, offsets, sorted_pairs, tile_offsets, tile_experts, tile_starts, pairs, E, block_m};
  return launch(K_DISPATCH, dim3(1), dim3(1024), 0, stream, a);
}

}  // extern "C"

// The forward pass enqueues both the expert-major and the grouped launches of
// a batch with few pairs per expert and lets the device pick (dsmoe_choose_path);
// while a PathScope is open, the four batch launchers below tag their
// arguments with the flag word and the value their workgroups need.
namespace {
struct PathSel {
  const uint32_t* path = nullptr;
  uint32_t mask = 0, want = 0;
};
thread_local PathSel t_path;
struct PathScope {
  PathScope(const uint32_t* p, uint32_t m, uint32_t w) { t_path = PathSel{p, m, w}; }
  ~PathScope() { t_path = PathSel{}; }
};
template <typename A>
void tag_path(A& a) {
  a.path = t_path.path;
  a.path_mask = t_path.mask;
  a.path_want = t_path.want;
}
}  // namespace

extern "C" {

// 1-D grid of the grouped kernels: ny slabs for each of 8 * ceil(tiles / 8)
// tile slots (the kernels' xcd_items mapping; it also covers the tiles x ny
// items of a grid with fewer than 8 tiles).
static unsigned xcd_grid(int tiles, int ny) { return 8u * (unsigned)((tiles + 7) / 8) * (unsigned)ny; }

int dsmoe_gate_up_mid_sorted(const void* gate, const void* up, const uint16_t* xh, const void* xq,
                             const uint32_t* sorted_pairs, const uint32_t* offsets, const uint32_t* tile_offsets,
                             const uint32_t* tile_experts, const uint32_t* tile_starts, const float* weights,
                             float* mid_out, int32_t d, int32_t I, int32_t k, int32_t E, int32_t pairs, float clamp,
                             dsmoe_stream_t stream) {
  if (!gate || !up || !xh || !xq || !sorted_pairs || !offsets || !tile_offsets || !tile_experts || !tile_starts ||
      !mid_out)
    return fail(DSMOE_ERR_INVALID, "gate_up_mid_sorted: null pointer");
  if (!aligned16(gate) || !aligned16(up) || !aligned16(xh))
    return fail(DSMOE_ERR_INVALID, "gate_up_mid_sorted: weights and xh must be 16-byte aligned");
  if (d <= 0 || d % 512 || d > 8192) return fail(DSMOE_ERR_UNSUPPORTED, "gate_up_mid_sorted: d must be a multiple of 512, <= 8192");
  if (I <= 0 || I % kGuBN || k <= 0 || E <= 0 || pairs < 0) return fail(DSMOE_ERR_INVALID, "gate_up_mid_sorted: bad shape");
  if (pairs == 0) return DSMOE_OK;
  GuGroupedArgs a{(const uint8_t*)gate, (const uint8_t*)up, xh, (const uint8_t*)xq, sorted_pairs, offsets,
                  tile_offsets, tile_experts, tile_starts, weights, mid_out, d, I, k, E, clamp};
  tag_path(a);
  // tiles per expert <= ceil(count / BM): at most pairs / BM + one partial tile per used expert
  const int max_tiles = pairs / kGuBM + std::min(E, pairs);
  return launch(K_GU_GROUPED, dim3(xcd_grid(max_tiles, I / kGuBN)), dim3(kGuThreads), 0, stream, a);
}

int dsmoe_down_sorted(const void* down, const int8_t* m8, const uint16_t* bsum_h, const void* mq,
                      const uint32_t* sorted_pairs, const uint32_t* offsets, const uint32_t* tile_offsets,
                      const uint32_t* tile_experts, const uint32_t* tile_starts, float* down_out, int32_t d, int32_t I,
                      int32_t E, int32_t pairs, dsmoe_stream_t stream) {
  if (!down || !m8 || !bsum_h || !mq || !sorted_pairs || !offsets || !tile_offsets || !tile_experts || !tile_starts ||
      !down_out)
    return fail(DSMOE_ERR_INVALID, "down_sorted: null pointer");
  if (!aligned16(down) || !aligned16(m8) || !aligned16(bsum_h))
    return fail(DSMOE_ERR_INVALID, "down_sorted: weights, m8 and bsum_h must be 16-byte aligned");
  if (d <= 0 || d % kDnBN || I <= 0 || I % 256 || E <= 0 || pairs < 0)
    return fail(DSMOE_ERR_INVALID, "down_sorted: bad shape");
  if (pairs == 0) return DSMOE_OK;
  DnGroupedArgs a{(const uint8_t*)down, m8, bsum_h, (const uint8_t*)mq, sorted_pairs, offsets, tile_offsets,
                  tile_experts, tile_starts, down_out, d, I, E};
  tag_path(a);
  const int max_tiles = pairs / kGuBM + std::min(E, pairs);
  return launch(K_DN_GROUPED, dim3(xcd_grid(max_tiles, d / kDnBN)), dim3(kDnThreads), 0, stream, a);
}

int dsmoe_gate_up_mid_em(const void* gate, const void* up, const void* xq, const uint32_t* sorted_pairs,
                         const uint32_t* offsets, const uint32_t* tile_offsets, const uint32_t* tile_experts,
                         const uint32_t* tile_starts, const float* weights, float* mid_out, int32_t d, int32_t I,
                         int32_t k, int32_t E, int32_t pairs, int32_t block_m, float clamp, dsmoe_stream_t stream) {
  if (!gate || !up || !xq || !sorted_pairs || !offsets || !tile_offsets || !tile_experts || !tile_starts || !mid_out)
    return fail(DSMOE_ERR_INVALID, "gate_up_mid_em: null pointer");
  if (!aligned16(gate) || !aligned16(up)) return fail(DSMOE_ERR_INVALID, "gate_up_mid_em: weights must be 16-byte aligned");
  if (I <= 0 || k <= 0 || E <= 0 || pairs < 0) return fail(DSMOE_ERR_INVALID, "gate_up_mid_em: bad shape");
  if (block_m < 1 || block_m > kEmPairs) return fail(DSMOE_ERR_INVALID, "gate_up_mid_em: block_m must be in 1..8");
  if (!up_rows_fits(d) || gate_up_em_lds(d / 256, block_m) > 64 * 1024)
    return fail(DSMOE_ERR_UNSUPPORTED, "gate_up_mid_em: d must be a multiple of 512 whose block_m activations fit 64 KB");
  if (pairs == 0) return DSMOE_OK;
  GuEmArgs m{};
  Shape sd;
  m.gu = gate_up_args(gate, up, xq, nullptr, weights, nullptr, nullptr, nullptr, mid_out, d, I, k, E, clamp, pairs, &sd);
  m.sorted_pairs = sorted_pairs;
  m.offsets = offsets;
  m.tile_offsets = tile_offsets;
  m.tile_experts = tile_experts;
  m.tile_starts = tile_starts;
  m.tiles = (I + 31) / 32;
  m.np = block_m;
  tag_path(m);
  const int64_t units = (int64_t)(pairs / block_m + std::min(E, pairs)) * m.tiles;
  if (units > 0x7FFFFFFF) return fail(DSMOE_ERR_UNSUPPORTED, "gate_up_mid_em: too many pairs");
  return launch(K_UP_EM, dim3((unsigned)units), dim3(256), gate_up_em_lds(d / 256, block_m), stream, m);
}

int dsmoe_down_em(const void* down, const void* mq, const uint32_t* sorted_pairs, const uint32_t* offsets,
                  const uint32_t* tile_offsets, const uint32_t* tile_experts, const uint32_t* tile_starts,
                  float* down_out, int32_t d, int32_t I, int32_t E, int32_t pairs, int32_t block_m,
                  dsmoe_stream_t stream) {
  if (!down || !mq || !sorted_pairs || !offsets || !tile_offsets || !tile_experts || !tile_starts || !down_out)
    return fail(DSMOE_ERR_INVALID, "down_em: null pointer");
  if (!aligned16(down)) return fail(DSMOE_ERR_INVALID, "down_em: weights must be 16-byte aligned");
  if (d <= 0 || I <= 0 || I % 256 || I > 2048 || E <= 0 || pairs < 0)
    return fail(I > 2048 ? DSMOE_ERR_UNSUPPORTED : DSMOE_ERR_INVALID, "down_em: bad shape (I a multiple of 256, <= 2048)");
  if (block_m < 1 || block_m > kEmPairs) return fail(DSMOE_ERR_INVALID, "down_em: block_m must be in 1..8");
  if (pairs == 0) return DSMOE_OK;
  DnEmArgs m{};
  Shape sd;
  m.dn = down_args(down, mq, nullptr, down_out, nullptr, d, I, 1, E, 1, &sd);
  m.sorted_pairs = sorted_pairs;
  m.offsets = offsets;
  m.tile_offsets = tile_offsets;
  m.tile_experts = tile_experts;
  m.tile_starts = tile_starts;
  m.tiles = (d + kDnEmRows - 1) / kDnEmRows;
  m.np = block_m;
  tag_path(m);
  const int64_t units = (int64_t)(pairs / block_m + std::min(E, pairs)) * m.tiles;
  if (units > 0x7FFFFFFF) return fail(DSMOE_ERR_UNSUPPORTED, "down_em: too many pairs");
  return launch(K_DN_EM, dim3((unsigned)units), dim3(256), down_em_lds(I / 256, block_m), stream, m);
}

}  // extern "C"

// Split over the row's lane classes for few token tiles: the smallest power
// of two (<= 8, and a whole number of stages of 8 / jmax class positions)
// that gives the launch at least `target` workgroups.
static int q80_ksplit(int T, int in_dim, int out_dim, bool two) {
  const int tiles = (T + kGuBM - 1) / kGuBM, ny = out_dim / (two ? 32 : 64);
  const int jmax = (in_dim / 32 + 31) / 32, G = 8 / jmax;
  int S = 1;
  const int target = two ? 512 : 256;  // measured on c3 and c4 (the down GEMM has a quarter of the K)
  while (S < 8 && (int64_t)tiles * ny * S < target && (32 / (2 * S)) % G == 0) S *= 2;
  return S;
}

// The shared expert's GEMM; with `part` (at least ksplit * T * cols floats)
// a split launch plus dsmoe_q80_combine when there are few token tiles.
static int q80_gemm_impl(const void* w0, const void* w1, const uint16_t* xh, const float* xscale, float* out,
                         int32_t in_dim, int32_t out_dim, int32_t T, float clamp, float* part, int32_t max_split,
                         dsmoe_stream_t stream) {
  if (!w0 || !xh || !xscale || !out) return fail(DSMOE_ERR_INVALID, "q8_0_gemm: null pointer");
  if (!aligned16(w0) || (w1 && !aligned16(w1)) || !aligned16(xh))
    return fail(DSMOE_ERR_INVALID, "q8_0_gemm: weights and xh must be 16-byte aligned");
  if (in_dim <= 0 || in_dim % 32 || in_dim > 8192 || T < 0 || out_dim <= 0 || out_dim % (w1 ? 32 : 64))
    return fail(DSMOE_ERR_UNSUPPORTED, "q8_0_gemm: in_dim a multiple of 32 (<= 8192), out_dim of 32 (two matrices) or 64");
  if (((size_t)(in_dim / 32) * Q8_0_BYTES) % 4) return fail(DSMOE_ERR_UNSUPPORTED, "q8_0_gemm: rows must be 4-byte multiples");
  if (T == 0) return DSMOE_OK;
  Q80GemmArgs a{(const uint8_t*)w0, (const uint8_t*)w1, xh, xscale, out, in_dim, out_dim, T, clamp};
  a.ksplit = part ? std::min(max_split, q80_ksplit(T, in_dim, out_dim, w1 != nullptr)) : 1;
  a.part = a.ksplit > 1 ? part : nullptr;
  // kernels specialised on the blocks per lane class, ceil(in_dim / 1024)
  const int jmax = (in_dim / 32 + 31) / 32;
  const Kern kern = jmax == 7 ? (w1 ? K_Q80_GEMM_SWIGLU_J7 : K_Q80_GEMM_J7)
                  : jmax == 2 ? (w1 ? K_Q80_GEMM_SWIGLU_J2 : K_Q80_GEMM_J2)
                              : (w1 ? K_Q80_GEMM_SWIGLU : K_Q80_GEMM);
  DSM_TRY(launch(kern, dim3(xcd_grid((T + kGuBM - 1) / kGuBM, out_dim / (w1 ? 32 : 64) * a.ksplit)), dim3(256), 0,
                 stream, a));
  if (a.ksplit == 1) return DSMOE_OK;
  Q80CombineArgs c{part, out, out_dim, T, a.ksplit, w1 ? 1 : 0, clamp};
  const int64_t n = (int64_t)T * out_dim;
  return launch(K_Q80_COMBINE, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, c);
}

extern "C" {

int dsmoe_q8_0_gemm(const void* w0, const void* w1, const uint16_t* xh, const float* xscale, float* out, int32_t in_dim,
                    int32_t out_dim, int32_t T, float clamp, dsmoe_stream_t stream) {
  return q80_gemm_impl(w0, w1, xh, xscale, out, in_dim, out_dim, T, clamp, nullptr, 1, stream);
}

// Shared expert for large batches: the Q8_0 matrices rewritten into the wide
// GEMM's operand layout once per call, then dsmoe_q80_wide[_swiglu] (blocks
// added in order; the exact kernels above keep the reference's tree).
// Batches of at least q80_wide_min_t() tokens take it: below that the grid of
// 128-token tiles is too small to fill the chip and the split exact kernel
// is faster.
static int q80_wide_min_t() { return 1024; }
static bool q80_wide_fits(int d, int Is) {
  return d % 128 == 0 && Is % 64 == 0 && d <= 8192 && Is <= 8192;
}
static int q80_unpack(const void* const* w, uint16_t* const* wh, float* const* ws, const int* rows, const int* nb, int n,
                      dsmoe_stream_t stream) {
  Q80UnpackArgs a{};
  unsigned units = 0;
  for (int m = 0; m < n; m++) {
    if (rows[m] % 16 || nb[m] % 2 || !aligned16(wh[m]) || (size_t)w[m] % 4)
      return fail(DSMOE_ERR_UNSUPPORTED, "q80_unpack: shape or alignment outside what the kernel assumes");
    a.w[m] = (const uint8_t*)w[m];
    a.wh[m] = wh[m];
    a.ws[m] = ws[m];
    a.rows[m] = rows[m];
    a.nb[m] = nb[m];
    units = std::max(units, (unsigned)(rows[m] / 16 * ((nb[m] + 15) / 16)));
  }
  return launch(K_Q80_UNPACK, dim3(units, (unsigned)n), dim3(256), 0, stream, a);
}
static int q80_wide_impl(const uint16_t* w0h, const float* w0s, const uint16_t* w1h, const float* w1s,
                         const uint16_t* xh, const float* xs, float* out, int in_dim, int out_dim, int T, float clamp,
                         dsmoe_stream_t stream) {
  const int rows = w1h ? kQwRowsSw : kQwRows;
  if (in_dim % 64 || out_dim % rows || T <= 0 || !aligned16(xh) || !aligned16(out))
    return fail(DSMOE_ERR_UNSUPPORTED, "q80_wide: shape or alignment outside what the kernel assumes");
  Q80WideArgs a{w0h, w0s, w1h, w1s, xh, xs, out, in_dim, out_dim, T, clamp};
  return launch(w1h ? K_Q80_WIDE_SW : K_Q80_WIDE, dim3(xcd_grid((T + kQwBT - 1) / kQwBT, out_dim / rows)),
                dim3(64 * kQwWaves), 0, stream, a);
}

extern "C" {

int dsmoe_q8_0_unpack(const void* w, int32_t rows, int32_t in_dim, uint16_t* codes, float* scales,
                      dsmoe_stream_t stream) {
  if (!w || !codes || !scales) return fail(DSMOE_ERR_INVALID, "q8_0_unpack: null pointer");
  if (rows <= 0 || rows % 16 || in_dim <= 0 || in_dim % 64)
    return fail(DSMOE_ERR_UNSUPPORTED, "q8_0_unpack: rows a multiple of 16, in_dim of 64");
  if (!aligned16(codes) || (uintptr_t)w % 4) return fail(DSMOE_ERR_INVALID, "q8_0_unpack: codes 16-byte, w 4-byte aligned");
  const void* ws[1] = {w};
  uint16_t* hs[1] = {codes};
  float* ss[1] = {scales};
  const int r[1] = {rows}, nb[1] = {in_dim / 32};
  return q80_unpack(ws, hs, ss, r, nb, 1, stream);
}

int dsmoe_q8_0_gemm_unpacked(const uint16_t* w0h, const float* w0s, const uint16_t* w1h, const float* w1s,
                             const uint16_t* xh, const float* xscale, float* out, int32_t in_dim, int32_t out_dim,
                             int32_t T, float clamp, dsmoe_stream_t stream) {
  if (!w0h || !w0s || !xh || !xscale || !out || (!w1h) != (!w1s))
    return fail(DSMOE_ERR_INVALID, "q8_0_gemm_unpacked: null pointer");
  if (!aligned16(w0h) || (w1h && !aligned16(w1h)) || !aligned16(xh) || !aligned16(out))
    return fail(DSMOE_ERR_INVALID, "q8_0_gemm_unpacked: codes, xh and out must be 16-byte aligned");
  if (in_dim <= 0 || in_dim % 64 || in_dim > 8192 || T < 0 || out_dim <= 0 || out_dim % (w1h ? kQwRowsSw : kQwRows))
    return fail(DSMOE_ERR_UNSUPPORTED,
                "q8_0_gemm_unpacked: in_dim a multiple of 64 (<= 8192), out_dim of 64 (two matrices) or 128");
  if (T == 0) return DSMOE_OK;
  return q80_wide_impl(w0h, w0s, w1h, w1s, xh, xscale, out, in_dim, out_dim, T, clamp, stream);
}

}  // extern "C"

// --------------------------------------------------------------------------
// Context + whole layer
// --------------------------------------------------------------------------
}  // extern "C"

struct dsmoe_ctx {
  dsmoe_config cfg;
  int32_t max_tokens;
  int device;
  size_t bytes = 0;
  std::vector<void*> allocs;
  float* logits = nullptr;
  int32_t* selected = nullptr;
  float* weights = nullptr;
  uint8_t* xq8k = nullptr;
  int8_t* xq80 = nullptr;
  float* xs80 = nullptr;
  float* mid = nullptr;
  uint8_t* midq = nullptr;
  float* sh_mid = nullptr;
  uint8_t* sh_midq = nullptr;
  int8_t* sh_q80 = nullptr;
  float* sh_s80 = nullptr;
  // grouped (sorted-by-expert) path for T > kDecodeMaxT
  uint16_t* xh = nullptr;        // Q8_K(x) qs as f16 [T][d]
  int8_t* m8 = nullptr;          // Q8_K(mid) qs as int8 [T*k][I]
  uint16_t* bsh = nullptr;       // Q8_K(mid) 16-element sums as f16 [T*k][I/16]
  uint16_t* xh80 = nullptr;      // Q8_0(x) codes as f16 [T][d]
  uint16_t* shh = nullptr;       // Q8_0(shared mid) codes as f16 [T][I_s]
  float* down_out = nullptr;     // [T*k][d]
  uint32_t* g_counts = nullptr;  // dispatch outputs
  uint32_t* g_offsets = nullptr;
  uint32_t* g_sorted = nullptr;
  uint32_t* g_tile_offsets = nullptr;
  uint32_t* g_tile_experts = nullptr;
  uint32_t* g_tile_starts = nullptr;
  // tiles of kGuBM pairs for the grouped down when the gate/up runs
  // expert-major (its tiles above are em_pairs() pairs)
  uint32_t* g_tile_offsets64 = nullptr;
  uint32_t* g_tile_experts64 = nullptr;
  uint32_t* g_tile_starts64 = nullptr;
  uint32_t* g_path = nullptr;  // dsmoe_choose_path's flags (expert-major or grouped, per launch)
  float* q80_part = nullptr;     // split shared-expert GEMM partials, [kQ80MaxSplit][min(T, 256)][cols]
  uint16_t* shw_h[3] = {};       // shared gate / up / down unpacked for dsmoe_q80_wide (codes as f16)
  // Batches on the wide shared-expert path run the quantization of x and the
  // shared expert's chain on `side` (default priority), forked before the
  // router and joined after the routed down: the quantization runs beside
  // the VALU-bound router, the shared GEMMs fill the routed grouped
  // launches' tails.  ev_xq orders the routed gate/up after the quantization.
  hipStream_t side = nullptr;
  hipEvent_t ev_fork = nullptr, ev_join = nullptr, ev_xq = nullptr;
  float* shw_s[3] = {};          // their block scales
  // hash routing (dsmoe_set_hash_routing): table [hash_rows][k], token ids [T]
  const int32_t* hash = nullptr;
  const int32_t* hash_tokens = nullptr;
  int32_t hash_rows = 0;
  // mid row counters of the fused mid quantization in dsmoe_up_rows:
  // [kMaxDecodeT*k*(I/256)] routed, then [kMaxDecodeT*ceil(I_s/256)] shared;
  // zero between launches (the workgroup completing a block resets its word)
  uint32_t* mid_cnt = nullptr;
  bool profiling = false;
  std::vector<hipEvent_t> event_pool;
  std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> pending;
  double stage_ms[DSMOE_STAGE_COUNT] = {};
  int64_t stage_launches[DSMOE_STAGE_COUNT] = {};
};

namespace {
template <class T>
int ctx_alloc(dsmoe_ctx* c, T** p, size_t bytes) {
  void* q = nullptr;
  bytes = std::max<size_t>(bytes, 16);
  hipError_t e = hipMalloc(&q, bytes);
  if (e != hipSuccess) return fail(DSMOE_ERR_NOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
  c->allocs.push_back(q);
  c->bytes += bytes;
  *p = (T*)q;
  return DSMOE_OK;
}
}  // namespace

// Brackets one forward stage with events when the context is profiling.
struct StageScope {
  dsmoe_ctx* c;
  int stage;
  hipStream_t s;
  hipEvent_t a = nullptr, b = nullptr;
  static hipEvent_t take(dsmoe_ctx* c) {
    if (!c->event_pool.empty()) {
      hipEvent_t e = c->event_pool.back();
      c->event_pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
  StageScope(dsmoe_ctx* c_, int stage_, dsmoe_stream_t s_) : c(c_), stage(stage_), s((hipStream_t)s_) {
    if (!c->profiling) return;
    a = take(c);
    b = take(c);
    if (a) (void)hipEventRecord(a, s);
  }
  ~StageScope() {
    if (!c->profiling || !a || !b) return;
    (void)hipEventRecord(b, s);
    c->pending.push_back({stage, {a, b}});
  }
};

extern "C" {

const char* dsmoe_stage_name(int32_t stage) {
  static const char* names[DSMOE_STAGE_COUNT] = {"prep", "select", "up", "midq", "dn",
                                                 "gu_grouped", "shared_up", "dn_grouped", "shared_dn"};
  return (stage >= 0 && stage < DSMOE_STAGE_COUNT) ? names[stage] : "?";
}

int dsmoe_set_hash_routing(dsmoe_ctx* c, const int32_t* hash, int32_t hash_rows, const int32_t* tokens) {
  if (!c) return fail(DSMOE_ERR_INVALID, "set_hash_routing: ctx is NULL");
  if (hash && hash_rows < 1) return fail(DSMOE_ERR_INVALID, "set_hash_routing: hash_rows < 1");
  c->hash = hash;
  c->hash_rows = hash ? hash_rows : 0;
  c->hash_tokens = hash ? tokens : nullptr;
  return DSMOE_OK;
}

int dsmoe_set_profiling(dsmoe_ctx* c, int32_t enable) {
  if (!c) return fail(DSMOE_ERR_INVALID, "set_profiling: ctx is NULL");
  c->profiling = enable != 0;
  return DSMOE_OK;
}

int dsmoe_profile_read(dsmoe_ctx* c, double* total_ms, int64_t* launches, int32_t reset) {
  if (!c) return fail(DSMOE_ERR_INVALID, "profile_read: ctx is NULL");
  for (auto& p : c->pending) {
    DSM_CHECK_HIP(hipEventSynchronize(p.second.second));
    float ms = 0.0f;
    DSM_CHECK_HIP(hipEventElapsedTime(&ms, p.second.first, p.second.second));
    c->stage_ms[p.first] += ms;
    c->stage_launches[p.first] += 1;
    c->event_pool.push_back(p.second.first);
    c->event_pool.push_back(p.second.second);
  }
  c->pending.clear();
  for (int i = 0; i < DSMOE_STAGE_COUNT; i++) {
    if (total_ms) total_ms[i] = c->stage_ms[i];
    if (launches) launches[i] = c->stage_launches[i];
    if (reset) { c->stage_ms[i] = 0; c->stage_launches[i] = 0; }
  }
  return DSMOE_OK;
}

}  // extern "C"

// Lays the matvec-path buffers of T tokens out from `base` (256-byte
// aligned, each rounded up to 256 bytes) and sets c's pointers to them;
// with base == nullptr only the size is computed.  Returns the bytes used.
static int layer_fits_lds(const dsmoe_config& cf) {
  if (gate_up_lds(cf.d_model / 256, 1) > 64 * 1024 || down_lds(cf.top_k, cf.d_ff / 256, 1) > 64 * 1024 ||
      (cf.shared_fmt == 0 && (q80_lds(cf.d_model / 32, 2, 1) > 64 * 1024 || q80_lds(cf.d_ff_shared / 32, 1, 1) > 64 * 1024)))
    return fail(DSMOE_ERR_UNSUPPORTED, "layer shape exceeds one workgroup's LDS");
  return DSMOE_OK;
}

static size_t carve_matvec(dsmoe_ctx* c, const dsmoe_config& cf, size_t T, uint8_t* base) {
  const size_t K = cf.top_k, E = cf.n_expert, d = cf.d_model, I = cf.d_ff, Is = std::max(cf.d_ff_shared, 256);
  size_t at = 0;
  auto C = [&](auto** p, size_t b) {
    using Ptr = std::remove_reference_t<decltype(*p)>;
    if (base) *p = (Ptr)(base + at);
    at += (std::max<size_t>(b, 16) + 255) & ~(size_t)255;
  };
  C(&c->logits, T * E * 4);
  C(&c->selected, T * K * 4);
  C(&c->weights, T * K * 4);
  C(&c->xq8k, T * (d / 256) * Q8K_BYTES);
  C(&c->xq80, T * d);
  C(&c->xs80, T * (d / 32) * 4);
  C(&c->mid, T * K * I * 4);
  C(&c->midq, T * K * (I / 256) * Q8K_BYTES);
  C(&c->sh_mid, T * Is * 4);
  C(&c->sh_midq, T * (Is / 256 + 1) * Q8K_BYTES);
  C(&c->sh_q80, T * Is);
  C(&c->sh_s80, T * (Is / 32 + 1) * 4);
  C(&c->mid_cnt, ((size_t)kMaxDecodeT * K * (I / 256) + (size_t)kMaxDecodeT * ((Is + 255) / 256)) * 4);
  return at;
}

extern "C" {

int dsmoe_create(const dsmoe_config* cfg, int32_t max_tokens, dsmoe_ctx** out) {
  if (!out) return fail(DSMOE_ERR_INVALID, "create: out is NULL");
  *out = nullptr;
  DSM_TRY(validate_cfg(cfg));
  if (max_tokens < 1) return fail(DSMOE_ERR_INVALID, "create: max_tokens must be >= 1");
  DSM_TRY(layer_fits_lds(*cfg));
  DeviceState* st = nullptr;
  DSM_TRY(load_device(nullptr, &st));
  dsmoe_ctx* c = new dsmoe_ctx();
  c->cfg = *cfg;
  c->max_tokens = max_tokens;
  if (hipGetDevice(&c->device) != hipSuccess) c->device = 0;
  const size_t T = (size_t)max_tokens, K = cfg->top_k, E = cfg->n_expert;
  const size_t d = cfg->d_model, I = cfg->d_ff, Is = std::max(cfg->d_ff_shared, 256);
  int rc = DSMOE_OK;
  auto A = [&](auto** p, size_t b) { if (rc == DSMOE_OK) rc = ctx_alloc(c, p, b); };
  uint8_t* base = nullptr;
  const size_t nbytes = carve_matvec(c, *cfg, T, nullptr);
  A(&base, nbytes);
  if (rc == DSMOE_OK) {
    carve_matvec(c, *cfg, T, base);
    if (hipMemset(base, 0, nbytes) != hipSuccess) rc = fail(DSMOE_ERR_HIP, "create: hipMemset of the scratch failed");
  }
  if (max_tokens > kDecodeMaxT && E <= 512) {
    const size_t P = T * K, max_tiles = P + std::min(E, P);  // dispatch tiles of any block_m >= 1
    A(&c->xh, T * d * 2);
    A(&c->m8, P * I);
    A(&c->bsh, P * (I / 16) * 2);
    A(&c->xh80, T * d * 2);
    A(&c->shh, T * Is * 2);
    A(&c->down_out, P * d * 4);
    A(&c->g_counts, E * 4);
    A(&c->g_offsets, (E + 1) * 4);
    A(&c->g_sorted, P * 4);
    A(&c->g_tile_offsets, (E + 1) * 4);
    A(&c->g_tile_experts, max_tiles * 4);
    A(&c->g_tile_starts, max_tiles * 4);
    const size_t max_tiles64 = P / kGuBM + std::min(E, P);
    A(&c->g_tile_offsets64, (E + 1) * 4);
    A(&c->g_tile_experts64, max_tiles64 * 4);
    A(&c->g_tile_starts64, max_tiles64 * 4);
    A(&c->g_path, 16);
    A(&c->q80_part, (size_t)kQ80MaxSplit * std::min<size_t>(T, 256) * std::max<size_t>(2 * Is, d) * 4);
    if (cfg->shared_fmt == 0 && q80_wide_fits((int)d, cfg->d_ff_shared) && max_tokens >= q80_wide_min_t()) {
      const size_t is = (size_t)cfg->d_ff_shared;
      for (int m = 0; m < 3; m++) {
        A(&c->shw_h[m], is * d * 2);
        A(&c->shw_s[m], is * d / 32 * 4);
      }
    }
    if (cfg->shared_fmt == 0 && rc == DSMOE_OK &&
        (hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking) != hipSuccess ||
         hipEventCreateWithFlags(&c->ev_fork, hipEventDisableTiming) != hipSuccess ||
         hipEventCreateWithFlags(&c->ev_join, hipEventDisableTiming) != hipSuccess ||
         hipEventCreateWithFlags(&c->ev_xq, hipEventDisableTiming) != hipSuccess))
      rc = fail(DSMOE_ERR_HIP, "create: side stream or events");
  }
  if (rc != DSMOE_OK) {
    std::string msg = g_err;
    dsmoe_destroy(c);
    return fail(rc, msg);
  }
  *out = c;
  return DSMOE_OK;
}

int dsmoe_destroy(dsmoe_ctx* c) {
  if (!c) return DSMOE_OK;
  for (auto& p : c->pending) {
    (void)hipEventSynchronize(p.second.second);
    c->event_pool.push_back(p.second.first);
    c->event_pool.push_back(p.second.second);
  }
  for (hipEvent_t e : c->event_pool) (void)hipEventDestroy(e);
  if (c->side) {
    (void)hipStreamSynchronize(c->side);
    (void)hipStreamDestroy(c->side);
  }
  if (c->ev_fork) (void)hipEventDestroy(c->ev_fork);
  if (c->ev_join) (void)hipEventDestroy(c->ev_join);
  if (c->ev_xq) (void)hipEventDestroy(c->ev_xq);
  for (void* p : c->allocs) (void)hipFree(p);
  delete c;
  return DSMOE_OK;
}

size_t dsmoe_scratch_bytes(const dsmoe_ctx* c) { return c ? c->bytes : 0; }

static int forward_impl(dsmoe_ctx* c, const dsmoe_weights* w, const float* x, int32_t T, float* shared_out,
                  float* routed_out, int32_t* selected, float* weights, dsmoe_stream_t stream) {
  if (!c || !w) return fail(DSMOE_ERR_INVALID, "forward: null pointer");
  if (T < 0 || T > c->max_tokens) return fail(DSMOE_ERR_INVALID, "forward: T outside 0..max_tokens");
  if (T == 0) return DSMOE_OK;  // no token: nothing is read or written (buffers of no rows may be null)
  if (!x || !routed_out) return fail(DSMOE_ERR_INVALID, "forward: null pointer");
  const dsmoe_config& cf = c->cfg;
  if (!w->router_f16 || !w->gate || !w->up || !w->down) return fail(DSMOE_ERR_INVALID, "forward: missing routed weights");
  if (cf.has_bias && !w->bias) return fail(DSMOE_ERR_INVALID, "forward: has_bias without bias");
  if (cf.shared_fmt >= 0 && (!w->sh_gate || !w->sh_up || !w->sh_down || !shared_out))
    return fail(DSMOE_ERR_INVALID, "forward: missing shared expert weights or output");
  const int d = cf.d_model, I = cf.d_ff, K = cf.top_k, Is = cf.d_ff_shared, E = cf.n_expert;
  int32_t* sel = selected ? selected : c->selected;
  float* wts = weights ? weights : c->weights;
  const int nb = d / 256, P = T * K;
  // Batches (T > 8, E <= 512: the dispatch sort's limit) run the routed
  // experts as grouped GEMMs over pairs sorted by expert; everything else
  // runs the matvec launches, one work item per (row tile, pair / token).
  const bool grouped = T > kDecodeMaxT && c->xh != nullptr;
  // Few pairs per expert (at most kEmMaxLoad on average): the routed experts
  // may stream their weights once per chunk of em_pairs() pairs
  // (expert-major matvec) instead of dequantizing them into MFMA tiles.
  // Both forms are enqueued and the device picks one from the sorted pairs
  // (dsmoe_choose_path): a skewed batch (a few experts holding most pairs)
  // runs grouped even at a low average load.
  const bool em = grouped && (int64_t)P <= (int64_t)kEmMaxLoad * E && em_fits(cf);
  // The int8 grouped down overtakes the expert-major one from about 2 pairs
  // per expert on average (c4, 4 per expert: 386 against 526 us), well before
  // the gate/up does.
  const bool dn_floor = (int64_t)P > (int64_t)kEmDnMaxLoad * E;
  // Large batches run the shared expert through the unpacked wide GEMM, over
  // the caller's unpacked matrices when the weights carry them (all six
  // pointers), else over the context's copies unpacked in this call.
  const bool wide = grouped && cf.shared_fmt == 0 && c->shw_h[0] != nullptr && T >= q80_wide_min_t();
  const bool pre_unpacked = w->sh_codes[0] && w->sh_codes[1] && w->sh_codes[2] && w->sh_scales[0] &&
                            w->sh_scales[1] && w->sh_scales[2];
  const uint16_t* const* shw_h = pre_unpacked ? w->sh_codes : (const uint16_t* const*)c->shw_h;
  const float* const* shw_s = pre_unpacked ? w->sh_scales : (const float* const*)c->shw_s;
  if (pre_unpacked && (!aligned16(w->sh_codes[0]) || !aligned16(w->sh_codes[1]) || !aligned16(w->sh_codes[2])))
    return fail(DSMOE_ERR_INVALID, "forward: unpacked shared-expert codes must be 16-byte aligned");
  // the shared expert's chain on the side stream (batches with a Q8_0 shared
  // expert); with
  // stage profiling on, every stage runs on the caller's stream so each
  // stage's time is its own
  const bool fork = grouped && cf.shared_fmt == 0 && c->side && !c->profiling;
  hipStream_t shs = fork ? c->side : (hipStream_t)stream;
  // In the row-streaming path the selection needs no launch of its own:
  // every routed gate/up workgroup runs it for its token.
  const bool up_rows = !grouped && up_rows_fits(d) && (cf.shared_fmt != 0 || q80_rows_fits(d));
  const bool fuse_sel = up_rows && !c->hash;
  if (fork) {
    if (hipEventRecord(c->ev_fork, (hipStream_t)stream) != hipSuccess ||
        hipStreamWaitEvent(c->side, c->ev_fork, 0) != hipSuccess)
      return fail(DSMOE_ERR_HIP, "forward: fork of the shared-expert stream");
  }
  // 1. router logits + Q8_K(x) + Q8_0(x)          (session.rs:1894-1909, 1991-2008, 2062-2073)
  {
    StageScope sc(c, DSMOE_STAGE_PREP, stream);
    RouterLogitsArgs r{(const uint16_t*)w->router_f16, x, c->logits, d, E, T};
    Q8KArgs q8k{x, c->xq8k, d, T, grouped ? c->xh : nullptr};
    Q80Args q80{x, c->xq80, c->xs80, d, T, grouped ? c->xh80 : nullptr};
    if (fork) {  // the router here, the quantizations on the side stream
      DSM_TRY(prep_impl(&r, nullptr, nullptr, stream));
      DSM_TRY(midq_impl(&q8k, nullptr, &q80, c->side));
      if (hipEventRecord(c->ev_xq, c->side) != hipSuccess)
        return fail(DSMOE_ERR_HIP, "forward: event after the quantization of x");
    } else {
      DSM_TRY(prep_impl(&r, &q8k, cf.shared_fmt == 0 ? &q80 : nullptr, stream));
    }
  }
  // 2. routing                                     (session.rs:2010-2058)
  if (!fuse_sel) {
    StageScope sc(c, DSMOE_STAGE_SELECT, stream);
    if (c->hash)  // hash routing (moe.rs:92-109): the token ids pick the experts
      DSM_TRY(dsmoe_router_select_hash(&cf, c->logits, c->hash, c->hash_rows, c->hash_tokens, 0, T, nullptr, sel,
                                       wts, stream));
    else
      DSM_TRY(dsmoe_router_select(&cf, c->logits, w->bias, T, nullptr, sel, wts, stream));
    if (grouped && !em)  // moe_count/prefix/scatter_sorted_pairs + tiles (moe.rs:299-362, 547-596)
      DSM_TRY(dsmoe_dispatch(sel, P, E, kGuBM, c->g_counts, c->g_offsets, c->g_sorted,
                             c->g_tile_offsets, c->g_tile_experts, c->g_tile_starts, stream));
    if (em) {  // the sort cut into em_pairs() and into 64-pair tiles, and the choice between the two
      DispatchArgs da{sel, c->g_counts, c->g_offsets, c->g_sorted, c->g_tile_offsets, c->g_tile_experts,
                      c->g_tile_starts, P, E, em_pairs()};
      da.tile_offsets2 = c->g_tile_offsets64;
      da.tile_experts2 = c->g_tile_experts64;
      da.tile_starts2 = c->g_tile_starts64;
      da.block_m2 = kGuBM;
      da.path_flags = c->g_path;
      da.dn_grouped = dn_floor ? 1 : 0;
      DSM_TRY(launch(K_DISPATCH, dim3(1), dim3(1024), 0, stream, da));
    }
  }
  // 3. routed + shared gate/up/SwiGLU              (session.rs:1910-1959, 2075-2112)
  // The row-streaming launch also quantizes the mid rows (step 4) when the
  // shared expert is Q8_0 or absent; its row counters cover kDecodeMaxT tokens.
  const bool fuse_midq = up_rows && T <= kDecodeMaxT &&
                         (cf.shared_fmt == -1 || (cf.shared_fmt == 0 && Is % 32 == 0));
  {
    StageScope sc(c, DSMOE_STAGE_UP, stream);
    UpArgs a{};
    Shape s1, s2{0, 64, 0};
    const int mb = 256;
    if (fuse_sel) {
      a.fuse_sel = 1;
      a.sel = RouterSelectArgs{c->logits, cf.has_bias ? w->bias : nullptr, nullptr, sel, wts, T, E, K,
                               cf.n_group > 1 ? cf.n_group : 1, cf.topk_group, cf.has_bias ? 1 : 0, cf.route_scale};
    }
    a.gu = gate_up_args(w->gate, w->up, c->xq8k, sel, wts, nullptr, nullptr, nullptr, c->mid, d, I, K, E,
                        cf.swiglu_clamp, P, &s1, mb);
    if (up_rows) { s1.R = kUpRowsR; s1.block = 256; s1.tiles = (I + kUpRowsR - 1) / kUpRowsR; }
    a.gu_tiles = s1.tiles;
    a.gu_work = grouped ? 0 : P;
    size_t lds = up_rows ? gate_up_rows_lds(nb) : gate_up_lds(nb, s1.R);
    if (fuse_sel) lds = std::max(lds, select_lds(E));
    if (fork && hipStreamWaitEvent((hipStream_t)stream, c->ev_xq, 0) != hipSuccess)
      return fail(DSMOE_ERR_HIP, "forward: wait for the quantization of x");
    if (em) {
      StageScope sg(c, DSMOE_STAGE_GU_GROUPED, stream);
      {
        PathScope ps(c->g_path, 1u, 0u);
        DSM_TRY(dsmoe_gate_up_mid_em(w->gate, w->up, c->xq8k, c->g_sorted, c->g_offsets, c->g_tile_offsets,
                                     c->g_tile_experts, c->g_tile_starts, wts, c->mid, d, I, K, E, P,
                                     em_pairs(), cf.swiglu_clamp, stream));
      }
      PathScope ps(c->g_path, 1u, 1u);
      DSM_TRY(dsmoe_gate_up_mid_sorted(w->gate, w->up, c->xh, c->xq8k, c->g_sorted, c->g_offsets,
                                       c->g_tile_offsets64, c->g_tile_experts64, c->g_tile_starts64, wts, c->mid, d,
                                       I, K, E, P, cf.swiglu_clamp, stream));
    } else if (grouped) {
      StageScope sg(c, DSMOE_STAGE_GU_GROUPED, stream);
      DSM_TRY(dsmoe_gate_up_mid_sorted(w->gate, w->up, c->xh, c->xq8k, c->g_sorted, c->g_offsets, c->g_tile_offsets,
                                       c->g_tile_experts, c->g_tile_starts, wts, c->mid, d, I, K, E, P,
                                       cf.swiglu_clamp, stream));
    }
    a.sh_fmt = cf.shared_fmt;
    if (cf.shared_fmt == 0) {
      a.sh_q80 = q80_args(w->sh_gate, w->sh_up, c->xq80, c->xs80, nullptr, nullptr, c->sh_mid, d, Is, T,
                          cf.swiglu_clamp, &s2, mb);
      lds = std::max(lds, q80_lds(d / 32, 2, s2.R));
    } else if (cf.shared_fmt == 1) {
      a.sh_iq2 = gate_up_args(w->sh_gate, w->sh_up, c->xq8k, nullptr, nullptr, nullptr, nullptr, nullptr, c->sh_mid,
                              d, Is, 1, 1, cf.swiglu_clamp, T, &s2, mb);
      lds = std::max(lds, gate_up_lds(nb, s2.R));
    }
    if (cf.shared_fmt >= 0) { a.sh_tiles = s2.tiles; a.sh_work = T; }
    if (up_rows && cf.shared_fmt == 0) {  // Q8_0 row-streaming tiles: 4 rows of gate and of up
      a.sh_tiles = q80_rows_tiles(Is, true);
      // the start delay of the shared expert's workgroups: for a shared
      // gate/up of 16 MB and more (c2: 31 MB), none below (c1: 6 MB)
      a.sh_delay = (int64_t)2 * Is * (d / 32) * 34 >= ((int64_t)16 << 20) ? 1 : 0;
      lds = std::max(lds, q80_rows_lds(d / 32));
    }
    if (grouped && cf.shared_fmt == 0) {  // shared expert as a GEMM over the whole batch
      a.sh_work = 0;
      StageScope sg(c, DSMOE_STAGE_SH_UP, shs);
      if (wide) {
        if (!pre_unpacked) {
          const void* ws[2] = {w->sh_gate, w->sh_up};
          const int rows[2] = {Is, Is}, nbs[2] = {d / 32, d / 32};
          DSM_TRY(q80_unpack(ws, c->shw_h, c->shw_s, rows, nbs, 2, shs));
        }
        DSM_TRY(q80_wide_impl(shw_h[0], shw_s[0], shw_h[1], shw_s[1], c->xh80, c->xs80, c->sh_mid, d, Is, T,
                              cf.swiglu_clamp, shs));
      } else {
        DSM_TRY(q80_gemm_impl(w->sh_gate, w->sh_up, c->xh80, c->xs80, c->sh_mid, d, Is, T, cf.swiglu_clamp,
                              T <= 256 ? c->q80_part : nullptr, kQ80MaxSplit, shs));
      }
    }
    if (fuse_midq) {
      a.fuse_midq = 1;
      a.midq = Q8KArgs{c->mid, c->midq, I, P};
      a.sh_midq = Q80Args{c->sh_mid, c->sh_q80, c->sh_s80, Is, T};
      a.mid_cnt = c->mid_cnt;
    }
    const int units = a.gu_tiles * a.gu_work + a.sh_tiles * a.sh_work;
    DSM_TRY(launch(up_rows ? K_UP_ROWS : K_UP, dim3(units), dim3(up_rows ? 256 : std::max(s1.block, s2.block)), lds,
                   stream, a));
  }
  // 4. Q8_K(mid) + Q8_0 / Q8_K of the shared mid  (session.rs:1964-1976, 2114-2127)
  if (!fuse_midq) {
    StageScope sc(c, DSMOE_STAGE_MIDQ, stream);
    Q8KArgs qa{c->mid, c->midq, I, P, nullptr, grouped ? c->m8 : nullptr, grouped ? c->bsh : nullptr};
    Q8KArgs qb{c->sh_mid, c->sh_midq, Is, T};
    Q80Args q80{c->sh_mid, c->sh_q80, c->sh_s80, Is, T, grouped ? c->shh : nullptr};
    if (fork) {  // the shared mid is quantized on the side stream
      DSM_TRY(midq_impl(&qa, nullptr, nullptr, stream));
      DSM_TRY(midq_impl(nullptr, nullptr, &q80, c->side));
    } else {
      DSM_TRY(midq_impl(&qa, cf.shared_fmt == 1 ? &qb : nullptr, cf.shared_fmt == 0 ? &q80 : nullptr, stream));
    }
  }
  // 5. routed down (+ slot sum) + shared down      (session.rs:1977-1986, 2129-2153)
  {
    StageScope sc(c, DSMOE_STAGE_DN, stream);
    DnArgs a{};
    Shape s1, s2{0, 64, 0};
    const bool rows = !grouped && dn_rows_fits(I, K) && (cf.shared_fmt != 0 || q80_rows_fits(Is));
    const int mb = rows ? 256 : 1024;
    a.dn = down_args(w->down, c->midq, sel, nullptr, routed_out, d, I, K, E, T, &s1, mb);
    a.dn_tiles = s1.tiles;
    a.dn_work = grouped ? 0 : T;
    if (grouped) {
      {
        StageScope sg(c, DSMOE_STAGE_DN_GROUPED, stream);
        if (em) {
          {
            PathScope ps(c->g_path, 2u, 0u);
            DSM_TRY(dsmoe_down_em(w->down, c->midq, c->g_sorted, c->g_offsets, c->g_tile_offsets,
                                  c->g_tile_experts, c->g_tile_starts, c->down_out, d, I, E, P, em_pairs(), stream));
          }
          PathScope ps(c->g_path, 2u, 2u);
          DSM_TRY(dsmoe_down_sorted(w->down, c->m8, c->bsh, c->midq, c->g_sorted, c->g_offsets, c->g_tile_offsets64,
                                    c->g_tile_experts64, c->g_tile_starts64, c->down_out, d, I, E, P, stream));
        } else {
          DSM_TRY(dsmoe_down_sorted(w->down, c->m8, c->bsh, c->midq, c->g_sorted, c->g_offsets, c->g_tile_offsets,
                                    c->g_tile_experts, c->g_tile_starts, c->down_out, d, I, E, P, stream));
        }
      }
      DSM_TRY(dsmoe_moe_sum(c->down_out, routed_out, d, K, T, stream));
    }
    size_t lds = down_lds(K, I / 256, s1.R);
    a.sh_fmt = cf.shared_fmt;
    if (cf.shared_fmt == 0) {
      a.sh_q80 = q80_args(w->sh_down, nullptr, c->sh_q80, c->sh_s80, shared_out, nullptr, nullptr, Is, d, T, 0.0f, &s2,
                          std::min(512, mb));
      lds = std::max(lds, q80_lds(Is / 32, 1, s2.R));
    } else if (cf.shared_fmt == 1) {
      a.sh_q2k = down_args(w->sh_down, c->sh_midq, nullptr, nullptr, shared_out, d, Is, 1, 1, T, &s2, mb);
      lds = std::max(lds, down_lds(1, Is / 256, s2.R));
    }
    if (cf.shared_fmt >= 0) { a.sh_tiles = s2.tiles; a.sh_work = T; }
    if (grouped && cf.shared_fmt == 0) {
      a.sh_work = 0;
      StageScope sg(c, DSMOE_STAGE_SH_DN, shs);
      if (wide) {
        if (!pre_unpacked) {
          const void* ws[1] = {w->sh_down};
          const int rows[1] = {d}, nbs[1] = {Is / 32};
          DSM_TRY(q80_unpack(ws, c->shw_h + 2, c->shw_s + 2, rows, nbs, 1, shs));
        }
        DSM_TRY(q80_wide_impl(shw_h[2], shw_s[2], nullptr, nullptr, c->shh, c->sh_s80, shared_out, Is, d, T, 0.0f,
                              shs));
      } else {
        DSM_TRY(q80_gemm_impl(w->sh_down, nullptr, c->shh, c->sh_s80, shared_out, Is, d, T, 0.0f,
                              T <= 256 ? c->q80_part : nullptr, kQ80MaxSplit, shs));
      }
    }
    if (rows) {
      a.dn_tiles = (d + kDnRowsR - 1) / kDnRowsR;
      lds = down_lds(K, I / 256, 0);
      if (cf.shared_fmt == 0) {
        a.sh_tiles = q80_rows_tiles(d, false);
        lds = std::max(lds, q80_rows_lds(Is / 32));
      } else if (cf.shared_fmt == 1) {
        lds = std::max(lds, down_lds(1, Is / 256, s2.R));
      }
    }
    DSM_TRY(launch(rows ? K_DN_ROWS : K_DN, dim3(a.dn_tiles * a.dn_work + a.sh_tiles * a.sh_work),
                   dim3(rows ? 256 : std::max(s1.block, s2.block)), lds, stream, a));
  }
  if (fork) {  // join: the caller's stream sees shared_out complete
    if (hipEventRecord(c->ev_join, c->side) != hipSuccess ||
        hipStreamWaitEvent((hipStream_t)stream, c->ev_join, 0) != hipSuccess)
      return fail(DSMOE_ERR_HIP, "forward: join of the shared-expert stream");
  }
  return DSMOE_OK;
}

int dsmoe_forward(dsmoe_ctx* c, const dsmoe_weights* w, const float* x, int32_t T, float* shared_out,
                  float* routed_out, int32_t* selected, float* weights, dsmoe_stream_t stream) {
  return forward_impl(c, w, x, T, shared_out, routed_out, selected, weights, stream);
}

int dsmoe_forward_noalloc(const dsmoe_config* cfg, const dsmoe_weights* w, const float* x, int32_t T,
                          float* shared_out, float* routed_out, int32_t* selected, float* weights,
                          dsmoe_stream_t stream) {
  DSM_TRY(validate_cfg(cfg));
  if (T < 0 || T > kDecodeMaxT) return fail(DSMOE_ERR_UNSUPPORTED, "forward_noalloc: T must be in 0..8");
  DSM_TRY(layer_fits_lds(*cfg));
  {
    // The first call on a device loads the code objects and clears the static
    // scratch (a launch and a synchronization), which a stream under graph
    // capture cannot take: that set-up must happen before capture.
    int dev = 0;
    DSM_CHECK_HIP(hipGetDevice(&dev));
    bool loaded = false;
    {
      std::lock_guard<std::mutex> lk(g_mu);
      loaded = dev >= 0 && dev < kMaxDevices && g_dev[dev].loaded;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (!loaded && hipStreamIsCapturing((hipStream_t)stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return fail(DSMOE_ERR_INVALID, "forward_noalloc: the device is not set up yet and the stream is capturing; "
                                     "call dsmoe_init (or one forward_noalloc) on this device before capture");
  }
  DeviceState* st = nullptr;
  DSM_TRY(load_device(nullptr, &st));
  dsmoe_ctx c;  // pointers into the static scratch; owns nothing
  c.cfg = *cfg;
  c.max_tokens = kDecodeMaxT;
  c.device = -1;
  const size_t need = carve_matvec(&c, *cfg, kDecodeMaxT, nullptr);
  if (need > st->noalloc_bytes)
    return fail(DSMOE_ERR_UNSUPPORTED, "forward_noalloc: the layer needs " + std::to_string(need) +
                                           " bytes of scratch; the static buffer holds " +
                                           std::to_string(st->noalloc_bytes));
  carve_matvec(&c, *cfg, kDecodeMaxT, st->noalloc);
  return forward_impl(&c, w, x, T, shared_out, routed_out, selected, weights, stream);
}

// --------------------------------------------------------------------------
// Synthetic tensors
// --------------------------------------------------------------------------
size_t dsmoe_tensor_bytes(int32_t fmt, int64_t n_mats, int32_t rows, int32_t cols) {
  if (n_mats < 0 || rows < 0 || cols < 0) return 0;
  const size_t per_row = fmt == DSMOE_FMT_IQ2_XXS ? (size_t)(cols + 255) / 256 * IQ2XXS_BYTES
                         : fmt == DSMOE_FMT_Q2_K  ? (size_t)(cols + 255) / 256 * Q2K_BYTES
                         : fmt == DSMOE_FMT_Q8_0  ? (size_t)(cols + 31) / 32 * Q8_0_BYTES
                         : fmt == DSMOE_FMT_F16   ? (size_t)cols * 2
                         : fmt == DSMOE_FMT_F32   ? (size_t)cols * 4
                                                  : 0;
  return per_row * (size_t)rows * (size_t)n_mats;
}

static int synth_check(int32_t fmt, int64_t n_mats, int32_t rows, int32_t cols, int32_t rows_real,
                       int32_t cols_real) {
  if (fmt < 0 || fmt > 4) return fail(DSMOE_ERR_INVALID, "synth: unknown format");
  if (n_mats < 1 || rows < 1 || cols < 1 || rows_real < 0 || cols_real < 0 || rows_real > rows || cols_real > cols)
    return fail(DSMOE_ERR_INVALID, "synth: bad shape");
  if ((fmt == DSMOE_FMT_IQ2_XXS || fmt == DSMOE_FMT_Q2_K) && cols % 256)
    return fail(DSMOE_ERR_INVALID, "synth: IQ2_XXS/Q2_K need cols % 256 == 0");
  if (fmt == DSMOE_FMT_Q8_0 && cols % 32) return fail(DSMOE_ERR_INVALID, "synth: Q8_0 needs cols % 32 == 0");
  return DSMOE_OK;
}

int dsmoe_synth_tensor(void* out, int32_t fmt, uint64_t seed, uint64_t tensor_id, int64_t n_mats, int32_t rows,
                       int32_t cols, int32_t rows_real, int32_t cols_real, float sigma, dsmoe_stream_t stream) {
  if (!out) return fail(DSMOE_ERR_INVALID, "synth: null pointer");
  DSM_TRY(synth_check(fmt, n_mats, rows, cols, rows_real, cols_real));
  DeviceState* st = nullptr;
  DSM_TRY(load_device(nullptr, &st));
  {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!st->d_lvlmap) {
      const auto& m = lvlmap_host();
      DSM_CHECK_HIP(hipMalloc(&st->d_lvlmap, m.size()));
      DSM_CHECK_HIP(hipMemcpy(st->d_lvlmap, m.data(), m.size(), hipMemcpyHostToDevice));
    }
  }
  const int per = fmt == DSMOE_FMT_Q8_0 ? 32 : 256;
  const int64_t total = n_mats * rows * (int64_t)((cols + per - 1) / per);
  SynthArgs a{(uint8_t*)out, st->d_lvlmap, seed, tensor_id, n_mats, rows, cols, rows_real, cols_real, sigma, fmt};
  const int64_t grid = (total + 255) / 256;
  if (grid > 0x7FFFFFFF) return fail(DSMOE_ERR_UNSUPPORTED, "synth: tensor too large");
  return launch(K_SYNTH, dim3((unsigned)grid), dim3(256), 0, stream, a);
}

int dsmoe_synth_tensor_host(void* out, int32_t fmt, uint64_t seed, uint64_t tensor_id, int64_t n_mats,
                            int32_t rows, int32_t cols, int32_t rows_real, int32_t cols_real, float sigma,
                            int32_t nthreads) {
  if (!out) return fail(DSMOE_ERR_INVALID, "synth_host: null pointer");
  DSM_TRY(synth_check(fmt, n_mats, rows, cols, rows_real, cols_real));
  const auto& lvl = lvlmap_host();
  const int per = fmt == DSMOE_FMT_Q8_0 ? 32 : 256;
  const int64_t bpr = (cols + per - 1) / per;
  const int64_t total = n_mats * rows * bpr;
  const uint64_t key = tensor_key(seed, tensor_id);
  auto work = [&](int64_t lo, int64_t hi) {
    float x[256];
    for (int64_t gid = lo; gid < hi; gid++) {
      const int64_t mat = gid / (rows * bpr);
      const int64_t rem = gid - mat * rows * bpr;
      const int row = (int)(rem / bpr);
      const int blk = (int)(rem - (int64_t)row * bpr);
      const int c0 = blk * per;
      const int n = std::min(per, cols - c0);
      for (int i = 0; i < per; i++)
        x[i] = i < n ? synth_value(key, mat, row, c0 + i, rows_real, cols_real, sigma) : 0.0f;
      uint8_t* o = (uint8_t*)out;
      switch (fmt) {
        case DSMOE_FMT_IQ2_XXS: iq2xxs_encode(x, o + gid * IQ2XXS_BYTES, lvl.data()); break;
        case DSMOE_FMT_Q2_K: q2k_encode(x, o + gid * Q2K_BYTES); break;
        case DSMOE_FMT_Q8_0: q8_0_encode(x, o + gid * Q8_0_BYTES); break;
        case DSMOE_FMT_F16: {
          uint16_t* p = (uint16_t*)out + (mat * rows + row) * (int64_t)cols + c0;
          for (int i = 0; i < n; i++) p[i] = f32_to_f16_rne(x[i]);
          break;
        }
        default: {
          float* p = (float*)out + (mat * rows + row) * (int64_t)cols + c0;
          for (int i = 0; i < n; i++) p[i] = x[i];
        }
      }
    }
  };
  int nt = std::max(1, std::min<int>(nthreads, 256));
  if (total < 64) nt = 1;
  std::vector<std::thread> th;
  for (int i = 1; i < nt; i++) th.emplace_back(work, total * i / nt, total * (i + 1) / nt);
  work(0, total / nt);
  for (auto& t : th) t.join();
  return DSMOE_OK;
}

}  // extern "C"
