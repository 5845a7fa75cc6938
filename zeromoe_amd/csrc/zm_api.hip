// zm_api.hip -- host side of libzeromoe_hip.so: the C ABI declared in
// include/zeromoe.h, argument validation, template dispatch and the per-device
// tables.  Everything below launches stream-ordered HIP work.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "../../include/zeromoe.h"
#include "zm_decode.hpp"
#include "zm_host.hpp"
#include "zm_mmq.hpp"

using namespace zm;

namespace {
thread_local char g_err[512] = "";
std::atomic<uint64_t> g_mmid_launches{0};
}  // namespace

int zm::fail(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return -1;
}
void zm::count_mmid_launch() { g_mmid_launches.fetch_add(1, std::memory_order_relaxed); }

namespace {

// ------------------------------------------------------------------ per-device state

constexpr int kMaxDevices = 16;

// Device-resident scratch of zm_mul_mat_id_static: one copy per GPU, held until
// the process ends.  Host code never passes `scratch` itself to a kernel (on the
// host the name is only a stand-in): its per-device address comes from
// hipGetSymbolAddress at set-up (DeviceState::scratch).
constexpr size_t kStaticScratchBytes = 16u << 20;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

struct DeviceState {
  bool ready = false;
  uint64_t *grid = nullptr;   // IQ2_XXS grid, 256 x u64
  uint64_t *signs = nullptr;  // 128 x u64 byte masks of ksigns_iq2xs
  uint64_t *iq4 = nullptr;    // IQ4_XS value table, 16 x i8
  uint64_t *iq3 = nullptr;    // IQ3_XXS grid, 256 x u32
  uint8_t *scratch = nullptr; // this device's address of `scratch`
  uint64_t *trace = nullptr;  // decode-kernel phase timestamps (ZEROMOE_TRACE=1)
  size_t trace_n = 0;
  int n_cu = 0;               // compute units
  // a dense shared expert runs beside the routed kernels of a multi-kernel
  // layer: forked from the caller's stream after x is quantized, joined
  // before the combine (default priority; the fork/join records into a HIP
  // graph like any other stream work)
  hipStream_t side = nullptr;
  hipEvent_t ev_fork = nullptr, ev_join = nullptr;
  std::mutex *fork_mu = nullptr;  // the events are per device: one fork at a time
};
DeviceState g_dev[kMaxDevices];
std::mutex g_mu;

void builtin_grid(uint64_t grid[256]) {
  // the 256 vectors of {1,3,5}^8 with an even digit sum ((v-1)/2 summed) of
  // smallest norm, lexicographic (coordinate 0 most significant) on ties;
  // coordinate bytes 1 -> 0x08, 3 -> 0x19, 5 -> 0x2b
  static const uint8_t bytev[3] = {0x08, 0x19, 0x2b};
  int count = 0;
  for (int norm = 0; norm < 200 && count < 256; ++norm)
    for (int idx = 0; idx < 6561 && count < 256; ++idx) {
      int t = idx, dig[8], sd = 0, nn = 0;
      for (int j = 7; j >= 0; --j) {
        dig[j] = t % 3;
        t /= 3;
      }
      for (int j = 0; j < 8; ++j) {
        sd += dig[j];
        nn += (1 + 2 * dig[j]) * (1 + 2 * dig[j]);
      }
      if ((sd & 1) || nn != norm) continue;
      uint64_t g = 0;
      for (int j = 0; j < 8; ++j) g |= (uint64_t)bytev[dig[j]] << (8 * j);
      grid[count++] = g;
    }
}

// ggml's kvalues_iq4nl (the table IQ4_NL / IQ4_XS index); replaceable with
// zm_set_iq4nl_table
void builtin_iq4nl(int8_t t[16]) {
  static const int8_t v[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
  for (int i = 0; i < 16; ++i) t[i] = v[i];
}

// stand-in IQ3_XXS grid: the 256 vectors of four 3-bit digits d with
// d0 + 2 d1 + 4 d2 + 8 d3 = 0 mod 16, in increasing order of the digit
// vector read as a base-8 number, digit d stored as the byte 4 + 8 d (62 for
// 7); ggml's own table is loaded with zm_set_iq3xxs_grid
void builtin_iq3_grid(uint32_t g[256]) {
  static const uint8_t lev[8] = {4, 12, 20, 28, 36, 44, 52, 62};
  int n = 0;
  for (int v = 0; v < 4096 && n < 256; ++v) {
    const int d0 = v & 7, d1 = (v >> 3) & 7, d2 = (v >> 6) & 7, d3 = (v >> 9) & 7;
    if ((d0 + 2 * d1 + 4 * d2 + 8 * d3) % 16) continue;
    g[n++] = (uint32_t)lev[d0] | ((uint32_t)lev[d1] << 8) | ((uint32_t)lev[d2] << 16) | ((uint32_t)lev[d3] << 24);
  }
}

int device_state(DeviceState **out) {
  int dev = 0;
  HIP_OK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail("device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState &d = g_dev[dev];
  if (!d.ready) {
    HIP_OK(hipDeviceGetAttribute(&d.n_cu, hipDeviceAttributeMultiprocessorCount, dev));
    HIP_OK(hipStreamCreateWithFlags(&d.side, hipStreamNonBlocking));
    HIP_OK(hipEventCreateWithFlags(&d.ev_fork, hipEventDisableTiming));
    HIP_OK(hipEventCreateWithFlags(&d.ev_join, hipEventDisableTiming));
    d.fork_mu = new std::mutex();
    uint64_t grid[256], signs[128];
    builtin_grid(grid);
    for (int i = 0; i < 128; ++i) {
      const int s = i | ((__builtin_popcount(i) & 1) << 7);  // ksigns_iq2xs
      uint64_t m = 0;
      for (int j = 0; j < 8; ++j)
        if ((s >> j) & 1) m |= 0xffull << (8 * j);
      signs[i] = m;
    }
    HIP_OK(hipMalloc(&d.grid, sizeof(grid)));
    HIP_OK(hipMalloc(&d.signs, sizeof(signs)));
    HIP_OK(hipMemcpy(d.grid, grid, sizeof(grid), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d.signs, signs, sizeof(signs), hipMemcpyHostToDevice));
    int8_t tab[16];
    builtin_iq4nl(tab);
    HIP_OK(hipMalloc(&d.iq4, 16));
    HIP_OK(hipMemcpy(d.iq4, tab, 16, hipMemcpyHostToDevice));
    uint32_t g3[256];
    builtin_iq3_grid(g3);
    HIP_OK(hipMalloc(&d.iq3, sizeof(g3)));
    HIP_OK(hipMemcpy(d.iq3, g3, sizeof(g3), hipMemcpyHostToDevice));
    void *sp = nullptr;
    HIP_OK(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)));
    d.scratch = (uint8_t *)sp;
    d.ready = true;
  }
  *out = &d;
  return 0;
}

// The state of the current device if zm_init (or any first call) has set it
// up; nullptr otherwise.  Allocates nothing.
DeviceState *device_state_if_ready() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_mu);
  return g_dev[dev].ready ? &g_dev[dev] : nullptr;
}

}  // namespace

int zm::device_grid(const uint64_t **grid) {
  DeviceState *d;
  if (device_state(&d)) return -1;
  *grid = d->grid;
  return 0;
}

int zm::device_table(int type, const uint64_t **table) {
  DeviceState *d;
  if (device_state(&d)) return -1;
  *table = type == T_IQ4_XS ? d->iq4 : (type == T_IQ3_XXS ? d->iq3 : d->grid);
  return 0;
}

namespace {

// ------------------------------------------------------------------ GEMV dispatch

template <int T, int LPR, int ITER, int NP, bool GU>
void launch_gemv_t(dim3 grid, const GemvArgs &a, hipStream_t st) {
  hipLaunchKernelGGL((k_gemv<T, LPR, ITER, NP, GU>), grid, dim3(256), 0, st, a);
}

template <int T, int NP, bool GU>
int launch_gemv_np(int U, dim3 grid, const GemvArgs &a, hipStream_t st) {
  if (U <= 16) launch_gemv_t<T, 16, 1, NP, GU>(grid, a, st);
  else if (U <= 32) launch_gemv_t<T, 32, 1, NP, GU>(grid, a, st);
  else if (U <= 64) launch_gemv_t<T, 64, 1, NP, GU>(grid, a, st);
  else if (U <= 128) launch_gemv_t<T, 64, 2, NP, GU>(grid, a, st);
  else if (U <= 192) launch_gemv_t<T, 64, 3, NP, GU>(grid, a, st);
  else if (U <= 256) launch_gemv_t<T, 64, 4, NP, GU>(grid, a, st);
  else return fail("row of %d blocks exceeds the 64-block limit", U / 4);
  return 0;
}

template <int T, bool GU>
int launch_gemv_type(int np, int U, dim3 grid, const GemvArgs &a, hipStream_t st) {
  if (np >= 4) return launch_gemv_np<T, 4, GU>(U, grid, a, st);
  if (np >= 2) return launch_gemv_np<T, 2, GU>(U, grid, a, st);
  return launch_gemv_np<T, 1, GU>(U, grid, a, st);
}

// true when the environment variable is set to "0" (switches a path off for testing)
bool getenv_flag_off(const char *name) {
  const char *e = getenv(name);
  return e && e[0] == '0';
}

bool type_supported(int t) {
  return t == T_Q2_K || t == T_Q3_K || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K || t == T_IQ2_XXS || t == T_IQ3_XXS ||
         t == T_IQ4_XS;
}

size_t row_bytes(int t, int64_t n) { return (size_t)(n / QK) * block_bytes(t); }

// pairs per bucket chunk held in registers
int pick_np(int n_pairs, int n_experts) {
  const int act = std::max(1, std::min(n_pairs, n_experts));
  const double avg = (double)n_pairs / act;
  return avg >= 3.0 ? 4 : (avg >= 1.5 ? 2 : 1);
}

// rows per workgroup: enough workgroups to cover the chip several times over
int pick_tile(int nrows, int U, int n_groups) {
  const int lpr = U <= 16 ? 16 : (U <= 32 ? 32 : 64);
  const int step = 4 * (64 / lpr);  // rows one workgroup covers per step
  const int target_wgs = 2048;
  const int tiles = std::max(1, target_wgs / std::max(1, n_groups));
  int tile = (nrows + tiles - 1) / tiles;
  tile = ((tile + step - 1) / step) * step;
  return std::max(step, tile);
}

int launch_gemv(int type, bool gateup, int np, const GemvArgs &a0, int n_groups, hipStream_t st) {
  GemvArgs a = a0;
  if ((type == T_IQ4_XS || type == T_IQ3_XXS) && device_table(type, &a.grid)) return -1;
  const int U = a.nb * 4;
  a.tile_rows = pick_tile(a.nrows, U, n_groups);
  dim3 grid((a.nrows + a.tile_rows - 1) / a.tile_rows, n_groups);
  int rc;
  switch (type) {
  case T_Q2_K: rc = gateup ? launch_gemv_type<T_Q2_K, true>(np, U, grid, a, st) : launch_gemv_type<T_Q2_K, false>(np, U, grid, a, st); break;
  case T_Q3_K: rc = gateup ? launch_gemv_type<T_Q3_K, true>(np, U, grid, a, st) : launch_gemv_type<T_Q3_K, false>(np, U, grid, a, st); break;
  case T_Q4_K: rc = gateup ? launch_gemv_type<T_Q4_K, true>(np, U, grid, a, st) : launch_gemv_type<T_Q4_K, false>(np, U, grid, a, st); break;
  case T_Q5_K: rc = gateup ? launch_gemv_type<T_Q5_K, true>(np, U, grid, a, st) : launch_gemv_type<T_Q5_K, false>(np, U, grid, a, st); break;
  case T_Q6_K: rc = gateup ? launch_gemv_type<T_Q6_K, true>(np, U, grid, a, st) : launch_gemv_type<T_Q6_K, false>(np, U, grid, a, st); break;
  case T_IQ3_XXS: rc = gateup ? launch_gemv_type<T_IQ3_XXS, true>(np, U, grid, a, st) : launch_gemv_type<T_IQ3_XXS, false>(np, U, grid, a, st); break;
  case T_IQ4_XS: rc = gateup ? launch_gemv_type<T_IQ4_XS, true>(np, U, grid, a, st) : launch_gemv_type<T_IQ4_XS, false>(np, U, grid, a, st); break;
  case T_IQ2_XXS: rc = gateup ? launch_gemv_type<T_IQ2_XXS, true>(np, U, grid, a, st) : launch_gemv_type<T_IQ2_XXS, false>(np, U, grid, a, st); break;
  default: return fail("unsupported weight type %d", type);
  }
  if (rc) return rc;
  HIP_OK(hipGetLastError());
  return 0;
}

// MFMA path for prefill-sized buckets: Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ3_XXS and IQ4_XS weights with at least 8
// pairs per active expert on average, Q2_K weights with at least 2.  a.items / a.n_items (or a.dense_S) must be set;
// max_items bounds *a.n_items.  Returns 1 when the path does not apply (the
// caller takes the GEMV path).
bool mmq_applies(int type, double avg_pairs) {
  return (((type == T_Q4_K || type == T_Q5_K || type == T_Q6_K || type == T_IQ4_XS || type == T_IQ2_XXS ||
            type == T_IQ3_XXS) &&
           avg_pairs >= 8.0) ||
          (type == T_Q2_K && avg_pairs >= 2.0)) &&
         !getenv_flag_off("ZEROMOE_MMQ");
}
// 16-token tiles per work item: routed buckets take 4 (the weight unpacking is
// shared by 64 pairs); Q2_K (small buckets of resident slots) and dense
// shared-expert rows 2
int mmq_tt(int type, bool dense) { return type != T_Q2_K && !dense ? 4 : 2; }
int launch_mmq(int type, bool gateup, const GemvArgs &a, int max_items, double avg_pairs, int tt, hipStream_t st,
               int nw = 4);
template <int T, int TT, int NW = 4>
void launch_mmq_t(bool gateup, dim3 grid, const GemvArgs &a, hipStream_t st) {
  grid.x = (unsigned)((a.nrows + 16 * NW - 1) / (16 * NW));  // NW waves of 16 weight rows per workgroup
  if (gateup)
    hipLaunchKernelGGL((k_mmq<T, true, TT, NW>), grid, dim3(64 * NW), 0, st, a);
  else
    hipLaunchKernelGGL((k_mmq<T, false, TT, NW>), grid, dim3(64 * NW), 0, st, a);
}
// tt: 16-token tiles per work item (the tiling the item list was cut with);
// nw: waves (16 weight rows each) per workgroup -- 1 for a Q4_K matrix whose
// 64-row tiles alone would leave most CUs idle (a dense shared expert)
int launch_mmq(int type, bool gateup, const GemvArgs &a, int max_items, double avg_pairs, int tt, hipStream_t st,
               int nw) {
  if (!mmq_applies(type, avg_pairs)) return 1;
  if ((size_t)a.nrows * a.w_rstride >= (1ull << 31) || max_items <= 0) return 1;
  const dim3 grid((unsigned)((a.nrows + 63) / 64), (unsigned)max_items);
  if (type == T_Q4_K) {
    if (tt == 8) {
      if (getenv_flag_off("ZEROMOE_MMQ_NW8")) launch_mmq_t<T_Q4_K, 8, 4>(gateup, grid, a, st);
      else launch_mmq_t<T_Q4_K, 8, 8>(gateup, grid, a, st);
    }
    else if (tt == 4) launch_mmq_t<T_Q4_K, 4>(gateup, grid, a, st);
    else if (nw == 1) launch_mmq_t<T_Q4_K, 2, 1>(gateup, grid, a, st);
    else launch_mmq_t<T_Q4_K, 2>(gateup, grid, a, st);
  } else if (type == T_Q5_K) {
    if (tt == 4) launch_mmq_t<T_Q5_K, 4>(gateup, grid, a, st);
    else launch_mmq_t<T_Q5_K, 2>(gateup, grid, a, st);
  } else if (type == T_IQ4_XS || type == T_IQ3_XXS || type == T_IQ2_XXS) {
    GemvArgs b = a;
    if (device_table(type, &b.grid)) return -1;
    if (type == T_IQ4_XS) {
      if (tt == 4) launch_mmq_t<T_IQ4_XS, 4>(gateup, grid, b, st);
      else launch_mmq_t<T_IQ4_XS, 2>(gateup, grid, b, st);
    } else if (type == T_IQ3_XXS) {
      if (tt == 4) launch_mmq_t<T_IQ3_XXS, 4>(gateup, grid, b, st);
      else launch_mmq_t<T_IQ3_XXS, 2>(gateup, grid, b, st);
    } else {
      if (tt == 4) launch_mmq_t<T_IQ2_XXS, 4>(gateup, grid, b, st);
      else launch_mmq_t<T_IQ2_XXS, 2>(gateup, grid, b, st);
    }
  } else if (type == T_Q6_K) {
    if (tt == 4) launch_mmq_t<T_Q6_K, 4>(gateup, grid, a, st);
    else launch_mmq_t<T_Q6_K, 2>(gateup, grid, a, st);
  } else {
    if (tt == 4) launch_mmq_t<T_Q2_K, 4>(gateup, grid, a, st);
    else launch_mmq_t<T_Q2_K, 2>(gateup, grid, a, st);
  }
  HIP_OK(hipGetLastError());
  return 0;
}
int mmq_max_items(int n_pairs, int n_experts) {
  return (n_pairs + MMQ_TOK - 1) / MMQ_TOK + std::min(n_pairs, n_experts);
}

int launch_quant(const float *x, size_t x_rstride, int nb, int rows, uint8_t *y, size_t y_rstride, int planar,
                 hipStream_t st) {
  if (rows <= 0) return 0;
  const long blocks = (long)rows * nb;  // 16 per workgroup
  hipLaunchKernelGGL(k_quant_q8K, dim3((unsigned)((blocks + 15) / 16)), dim3(256), 0, st, x, x_rstride, nb, rows, y,
                     y_rstride, planar);
  HIP_OK(hipGetLastError());
  return 0;
}

// simple bump allocator over a caller workspace
struct Bump {
  uint8_t *base;
  size_t off = 0;
  template <class P>
  P *take(size_t bytes) {
    off = (off + 255) & ~(size_t)255;
    P *p = reinterpret_cast<P *>(base ? base + off : nullptr);
    off += bytes;
    return p;
  }
};

}  // namespace

// ====================================================================== C ABI

extern "C" {

const char *zm_last_error(void) { return g_err; }
const char *zm_version(void) { return "zeromoe_amd 0.1 (gfx950)"; }

int zm_init(void) {
  DeviceState *d;
  return device_state(&d);
}

void zm_iq2xxs_builtin_grid(uint64_t grid[256]) { builtin_grid(grid); }

int zm_set_iq2xxs_grid(const uint64_t grid[256]) {
  DeviceState *d;
  if (device_state(&d)) return -1;
  HIP_OK(hipMemcpy(d->grid, grid, 256 * sizeof(uint64_t), hipMemcpyHostToDevice));
  return 0;
}

void zm_iq4nl_builtin_table(int8_t table[16]) { builtin_iq4nl(table); }

void zm_iq3xxs_builtin_grid(uint32_t grid[256]) { builtin_iq3_grid(grid); }

int zm_set_iq3xxs_grid(const uint32_t grid[256]) {
  DeviceState *d;
  if (device_state(&d)) return -1;
  HIP_OK(hipMemcpy(d->iq3, grid, 256 * sizeof(uint32_t), hipMemcpyHostToDevice));
  return 0;
}

int zm_set_iq4nl_table(const int8_t table[16]) {
  DeviceState *d;
  if (device_state(&d)) return -1;
  HIP_OK(hipMemcpy(d->iq4, table, 16, hipMemcpyHostToDevice));
  return 0;
}

int zm_mul_mat_id_negative_skip(void) { return 1; }
int zm_mul_mat_id_negative_skip_batched(void) { return 1; }
uint64_t zm_mul_mat_id_launches(void) { return g_mmid_launches.load(std::memory_order_relaxed); }

int zm_quantize_q8_K(const float *x, int64_t rows, int64_t n, void *y, void *stream) {
  if (!x || !y || rows < 0 || n <= 0 || n % QK) return fail("zm_quantize_q8_K: bad arguments");
  return launch_quant(x, (size_t)n, (int)(n / QK), (int)rows, (uint8_t *)y, (size_t)(n / QK) * 292, 0,
                      (hipStream_t)stream);
}

int zm_router(const zm_router_spec *spec, const float *logits, const float *logit_bias, const float *sel_bias,
              const int32_t *route_map, const float *route_mask, int S, int32_t *ids, float *weights,
              void *stream) {
  if (!spec || !logits || !ids || !weights || S < 0) return fail("zm_router: null argument");
  if (spec->n_experts <= 0 || spec->n_experts > ROUTER_MAX_E) return fail("zm_router: n_experts out of range");
  if (spec->topk <= 0 || spec->topk > spec->n_experts || spec->topk > 64) return fail("zm_router: bad topk");
  if (spec->n_groups > 64) return fail("zm_router: n_groups > 64");
  if (spec->gating < 0 || spec->gating > 2) return fail("zm_router: bad gating");
  if (S == 0) return 0;
  RouterArgs a{logits, logit_bias, sel_bias, route_map, route_mask, spec->n_experts, spec->topk, spec->gating,
               spec->n_groups, spec->n_groups_used, spec->weights_norm, spec->weights_scale, ids, weights};
  hipLaunchKernelGGL(k_router, dim3((S + 3) / 4), dim3(256), 0, (hipStream_t)stream, a, S);
  HIP_OK(hipGetLastError());
  return 0;
}

int zm_bucket(const int32_t *ids, int S, int K, int E, int32_t *counts, int32_t *offs, int32_t *pairs,
              int32_t *active, int32_t *n_active, void *stream) {
  if (!ids || !counts || !offs || !pairs || !active || !n_active) return fail("zm_bucket: null argument");
  if (E <= 0 || E > BUCKET_MAX_E) return fail("zm_bucket: E out of range (1..%d)", BUCKET_MAX_E);
  if (S < 0 || K <= 0) return fail("zm_bucket: bad S/K");
  hipLaunchKernelGGL(k_bucket, dim3(1), dim3(1024), 0, (hipStream_t)stream, ids, S * K, E, counts, offs, pairs,
                     active, n_active);
  HIP_OK(hipGetLastError());
  return 0;
}

// ---------------------------------------------------------------- mul_mat_id hook

}  // extern "C"

namespace {

// A validated MUL_MAT_ID shape (see zm_mul_mat_id's rules) and the workspace
// it needs: planar Q8_K rows of src1, a contiguous copy of ids, the bucket
// arrays and the MFMA work list.
struct MmidShape {
  int64_t I, O, E, n_ids, S, ne11, n_pairs, nq;
  int nb;
  size_t ws_bytes;
};

struct MmidWs {
  uint8_t *xq;
  int32_t *idc, *counts, *offs, *pairs, *active, *n_active, *items, *n_items;
};

size_t mmid_carve(const MmidShape &m, uint8_t *base, MmidWs *out) {
  Bump b{base};
  MmidWs w{};
  w.xq = b.take<uint8_t>((size_t)m.nq * q8_row_bytes(m.nb));
  w.idc = b.take<int32_t>((size_t)m.n_pairs * 4);
  w.counts = b.take<int32_t>((size_t)m.E * 4);
  w.offs = b.take<int32_t>((size_t)(m.E + 1) * 4);
  w.pairs = b.take<int32_t>((size_t)m.n_pairs * 4);
  w.active = b.take<int32_t>((size_t)m.E * 4);
  w.n_active = b.take<int32_t>(4);
  w.items = b.take<int32_t>((size_t)mmq_max_items((int)m.n_pairs, (int)m.E) * 4);
  w.n_items = b.take<int32_t>(4);
  if (out) *out = w;
  return b.off + 256;
}

// The validation rules of the reference hook (kquant_matmul.cu:705-722) plus
// this kernel set's limits; false = decline.
bool mmid_shape(const zm_tensor *w, const zm_tensor *x, const zm_tensor *ids, const zm_tensor *y, MmidShape *m) {
  if (!w || !x || !ids || !y) return false;
  if (!type_supported(w->type) || x->type != T_F32 || y->type != T_F32 || ids->type != T_I32) return false;
  const int64_t I = w->ne[0], O = w->ne[1], E = w->ne[2];
  if (I <= 0 || I % QK || I / QK > 64 || O <= 0 || O > INT32_MAX || E <= 0 || E > BUCKET_MAX_E || w->ne[3] != 1)
    return false;
  if (w->nb[1] != row_bytes(w->type, I) || w->nb[2] < (size_t)O * w->nb[1]) return false;
  const int64_t n_ids = ids->ne[0], S = ids->ne[1];
  if (ids->nb[0] != 4 || n_ids <= 0 || S <= 0 || ids->ne[2] != 1 || ids->ne[3] != 1) return false;
  if (x->nb[0] != 4 || x->ne[0] != I || (x->ne[1] != 1 && x->ne[1] != n_ids) || x->ne[2] != S || x->ne[3] != 1)
    return false;
  if (x->nb[1] % 16 || x->nb[2] % 16 || ((uintptr_t)x->data & 15)) return false;  // float4 row loads
  if (y->nb[0] != 4 || y->ne[0] != O || y->ne[1] != n_ids || y->ne[2] != S || y->ne[3] != 1) return false;
  if (y->nb[1] % 4 || y->nb[2] % 4 || ids->nb[1] % 4) return false;
  const int64_t n_pairs = n_ids * S;
  if (n_pairs > (1 << 24)) return false;
  m->I = I;
  m->O = O;
  m->E = E;
  m->n_ids = n_ids;
  m->S = S;
  m->ne11 = x->ne[1];
  m->n_pairs = n_pairs;
  m->nq = m->ne11 * S;
  m->nb = (int)(I / QK);
  m->ws_bytes = mmid_carve(*m, nullptr, nullptr);
  return true;
}

// The op on a workspace of at least m.ws_bytes (256-byte aligned); launches
// only, stream-ordered, allocates nothing.  Returns 1 handled / 0 failed.
int mmid_exec(const MmidShape &m, const zm_tensor *w, const zm_tensor *x, const zm_tensor *ids, zm_tensor *y,
              hipStream_t st, uint8_t *ws, const DeviceState *d) {
  MmidWs b;
  mmid_carve(m, ws, &b);
  const int nb = m.nb;
  const int ne11 = (int)m.ne11;
  const int64_t S = m.S, n_ids = m.n_ids, n_pairs = m.n_pairs, nq = m.nq, E = m.E, O = m.O;
  // 1. quantize src1 rows (token t, row i11) -> planar Q8_K row t*ne11 + i11
  if (x->nb[2] == (size_t)ne11 * x->nb[1]) {
    if (launch_quant((const float *)x->data, x->nb[1] / 4, nb, (int)nq, b.xq, q8_row_bytes(nb), 1, st)) return 0;
  } else {
    for (int64_t t = 0; t < S; ++t) {
      const float *xt = (const float *)((const char *)x->data + t * x->nb[2]);
      if (launch_quant(xt, x->nb[1] / 4, nb, ne11, b.xq + (size_t)t * ne11 * q8_row_bytes(nb), q8_row_bytes(nb), 1,
                       st))
        return 0;
    }
  }
  // 2. ids -> contiguous [S][n_ids] (strided copy), then bucket
  if (ids->nb[1] == (size_t)n_ids * 4) {
    if (hipMemcpyAsync(b.idc, ids->data, (size_t)n_pairs * 4, hipMemcpyDeviceToDevice, st) != hipSuccess) return 0;
  } else {
    if (hipMemcpy2DAsync(b.idc, (size_t)n_ids * 4, ids->data, ids->nb[1], (size_t)n_ids * 4, (size_t)S,
                         hipMemcpyDeviceToDevice, st) != hipSuccess)
      return 0;
  }
  hipLaunchKernelGGL(k_bucket, dim3(1), dim3(1024), 0, st, b.idc, (int)n_pairs, (int)E, b.counts, b.offs, b.pairs,
                     b.active, b.n_active);
  // 3. skipped / invalid routes (pairs over grid x and y, each <= 65535)
  {
    const unsigned gy = (unsigned)std::min<int64_t>(n_pairs, 65535);
    hipLaunchKernelGGL(k_fill_skipped, dim3((unsigned)std::min<int64_t>((O + 255) / 256, 64), gy), dim3(256), 0, st,
                       b.idc, (size_t)n_ids, (size_t)1, (int)n_ids, (int)S, (int)E, (int)O, (float *)y->data,
                       y->nb[2] / 4, y->nb[1] / 4);
  }
  // 4. bucketed GEMV or MFMA
  GemvArgs a{};
  a.w0 = (const uint8_t *)w->data;
  a.w_estride = w->nb[2];
  a.w_rstride = w->nb[1];
  a.nrows = (int)O;
  a.nb = nb;
  a.xq = b.xq;
  a.xq_rstride = q8_row_bytes(nb);
  a.ne11 = ne11;
  a.K = (int)n_ids;
  a.n_active = b.n_active;
  a.active = b.active;
  a.offs = b.offs;
  a.pairs = b.pairs;
  a.out = (float *)y->data;
  a.out_s = y->nb[2] / 4;
  a.out_k = y->nb[1] / 4;
  a.grid = d->grid;
  a.signs = d->signs;
  const int groups = (int)std::min<int64_t>(E, n_pairs);
  {
    // the MFMA path addresses the activations through a 32-bit buffer offset
    const double avg = (size_t)nq * q8_row_bytes(nb) < (1ull << 31) ? (double)n_pairs / groups : 0.0;
    if (mmq_applies(w->type, avg))
      hipLaunchKernelGGL(k_mmq_items, dim3(1), dim3(1024), 0, st, b.n_active, b.active, b.offs, b.items, b.n_items,
                         16 * mmq_tt(w->type, false));
    a.items = b.items;
    a.n_items = b.n_items;
    a.xq_bytes = (uint32_t)((size_t)nq * q8_row_bytes(nb));
    const int rc = launch_mmq(w->type, false, a, mmq_max_items((int)n_pairs, (int)E), avg, mmq_tt(w->type, false), st);
    if (rc < 0 || (rc > 0 && launch_gemv(w->type, false, pick_np((int)n_pairs, (int)E), a, groups, st))) return 0;
  }
  count_mmid_launch();
  return hipPeekAtLastError() == hipSuccess ? 1 : 0;
}

// Caller-owned workspaces bound to (device, stream) by zm_mul_mat_id_set_workspace.
struct WsBinding {
  int dev;
  hipStream_t stream;
  uint8_t *ptr;
  size_t bytes;
};
constexpr int kMaxBindings = 64;
WsBinding g_bind[kMaxBindings];
int g_nbind = 0;
std::mutex g_bind_mu;

}  // namespace

extern "C" {

size_t zm_mul_mat_id_workspace_size(const zm_tensor *src0, const zm_tensor *src1, const zm_tensor *ids,
                                    const zm_tensor *dst) {
  MmidShape m;
  return mmid_shape(src0, src1, ids, dst, &m) ? m.ws_bytes : 0;
}

int zm_mul_mat_id_set_workspace(void *stream, void *workspace, size_t bytes) {
  int dev = 0;
  HIP_OK(hipGetDevice(&dev));
  if (workspace && ((uintptr_t)workspace & 255)) return fail("zm_mul_mat_id_set_workspace: workspace not 256-byte aligned");
  std::lock_guard<std::mutex> lk(g_bind_mu);
  for (int i = 0; i < g_nbind; ++i)
    if (g_bind[i].dev == dev && g_bind[i].stream == (hipStream_t)stream) {
      if (workspace) {
        g_bind[i].ptr = (uint8_t *)workspace;
        g_bind[i].bytes = bytes;
      } else {
        g_bind[i] = g_bind[--g_nbind];
      }
      return 0;
    }
  if (!workspace) return 0;
  if (g_nbind == kMaxBindings) return fail("zm_mul_mat_id_set_workspace: more than %d bound streams", kMaxBindings);
  g_bind[g_nbind++] = WsBinding{dev, (hipStream_t)stream, (uint8_t *)workspace, bytes};
  return 0;
}

int zm_mul_mat_id(const zm_tensor *w, const zm_tensor *x, const zm_tensor *ids, zm_tensor *y, void *stream,
                  int execute) {
  MmidShape m;
  if (!mmid_shape(w, x, ids, y, &m)) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  uint8_t *ws = nullptr;
  {
    // query: the smallest workspace bound on this device must hold the shape
    // (ggml asks with no stream, then executes on one of its streams);
    // execute: the workspace bound to this stream
    std::lock_guard<std::mutex> lk(g_bind_mu);
    size_t cap = 0;
    bool any = false;
    for (int i = 0; i < g_nbind; ++i) {
      if (g_bind[i].dev != dev) continue;
      if (!execute) {
        cap = any ? std::min(cap, g_bind[i].bytes) : g_bind[i].bytes;
        any = true;
      } else if (g_bind[i].stream == (hipStream_t)stream) {
        cap = g_bind[i].bytes;
        ws = g_bind[i].ptr;
        any = true;
      }
    }
    if (!any || cap < m.ws_bytes) {
      fail("zm_mul_mat_id: %s (needs %zu bytes, zm_mul_mat_id_workspace_size)",
           any ? "bound workspace too small" : "no workspace bound for this device/stream", m.ws_bytes);
      return 0;
    }
  }
  if (!execute) return 1;
  DeviceState *d;
  if (device_state(&d)) return 0;
  return mmid_exec(m, w, x, ids, y, (hipStream_t)stream, ws, d);
}

int zm_mul_mat_id_static(const zm_tensor *w, const zm_tensor *x, const zm_tensor *ids, zm_tensor *dst, void *stream,
                         int execute) {
  MmidShape m;
  if (!mmid_shape(w, x, ids, dst, &m)) return 0;
  if (m.ws_bytes > kStaticScratchBytes) {
    fail("zm_mul_mat_id_static: shape needs %zu bytes of scratch, more than the %zu-byte device array", m.ws_bytes,
         kStaticScratchBytes);
    return 0;
  }
  if (!execute) return 1;
  DeviceState *d = device_state_if_ready();
  if (!d) {
    fail("zm_mul_mat_id_static: zm_init has not run on this device");
    return 0;
  }
  // every scratch array is written before it is read within the call, so
  // nothing needs clearing between calls
  return mmid_exec(m, w, x, ids, dst, (hipStream_t)stream, d->scratch, d);
}

// ---------------------------------------------------------------- debug: block dots

}  // extern "C"

namespace {
// Debug kernel: per super-block integer parts of one weight row against one
// Q8_K row, computed by both decode dot paths -- the 4-lane quarter path of the
// bucketed GEMV and the whole-block unit path of the fused decode kernel.  The
// unit result is written; a disagreement writes INT32_MIN into isum instead.
template <int T>
__global__ void k_block_dots(const uint8_t *w, const uint8_t *xq, int nb, int32_t *isum, int32_t *imin,
                             const uint64_t *grid, const uint64_t *signs) {
  const int lane = threadIdx.x & 63;
  const int gq = blockIdx.x * 64 + lane;  // quarter index
  const int b = gq >> 2, q = gq & 3;
  QInt r{0, 0};
  int ui = 0, um = 0;
  if (b < nb) {
    Q8Slice s;
    WSlice ws;
    load_q8_slice<T>(xq, nb, b, q, s);
    load_w_slice<T>(w + (size_t)b * block_bytes(T), q, ws);
    r = quarter_int<T>(ws, q, s, grid, signs);
    if constexpr (has_unit<T>()) {
      if (q < unit_per_block<T>()) {
        const rsrc_t rw = make_rsrc(w, (uint32_t)(nb * block_bytes(T)));
        Unit<T> u[1];
        load_unit<T>(rw, b * block_bytes(T), q, u[0]);
        int ri[1], rm[1];
        unit_ints<T, 1>(u, q, xblk_planar(xq, nb, b), grid, signs, ri, rm);
        ui = ri[0];
        um = rm[0];
      }
    }
  }
  r.isum = group_sum_i<4>(r.isum);
  r.imin = group_sum_i<4>(r.imin);
  if constexpr (has_unit<T>()) {
    ui = group_sum_i<4>(ui);
    um = group_sum_i<4>(um);
  } else {
    ui = r.isum;  // no whole-block path for this type: the quarter sums are reported
    um = r.imin;
  }
  if (b < nb && q == 0) {
    const bool agree = ui == r.isum && um == r.imin;
    isum[b] = agree ? ui : INT32_MIN;
    imin[b] = um;
  }
}
}  // namespace

extern "C" {

int zm_block_dots(int type, const void *w_row, const float *x, int n, int32_t *isum, int32_t *imin, void *stream) {
  if (!type_supported(type) || n <= 0 || n % QK || !w_row || !x || !isum || !imin)
    return fail("zm_block_dots: bad arguments");
  DeviceState *d;
  if (device_state(&d)) return -1;
  hipStream_t st = (hipStream_t)stream;
  const int nb = n / QK;
  uint8_t *xq = nullptr;
  HIP_OK(hipMallocAsync((void **)&xq, q8_row_bytes(nb), st));
  if (launch_quant(x, (size_t)n, nb, 1, xq, q8_row_bytes(nb), 1, st)) return -1;
  const dim3 g((unsigned)((nb * 4 + 63) / 64));
  const uint8_t *w = (const uint8_t *)w_row;
  switch (type) {
  case T_Q2_K: hipLaunchKernelGGL(k_block_dots<T_Q2_K>, g, dim3(64), 0, st, w, xq, nb, isum, imin, d->grid, d->signs); break;
  case T_Q3_K: hipLaunchKernelGGL(k_block_dots<T_Q3_K>, g, dim3(64), 0, st, w, xq, nb, isum, imin, d->grid, d->signs); break;
  case T_Q4_K: hipLaunchKernelGGL(k_block_dots<T_Q4_K>, g, dim3(64), 0, st, w, xq, nb, isum, imin, d->grid, d->signs); break;
  case T_Q5_K: hipLaunchKernelGGL(k_block_dots<T_Q5_K>, g, dim3(64), 0, st, w, xq, nb, isum, imin, d->grid, d->signs); break;
  case T_Q6_K: hipLaunchKernelGGL(k_block_dots<T_Q6_K>, g, dim3(64), 0, st, w, xq, nb, isum, imin, d->grid, d->signs); break;
  case T_IQ4_XS: hipLaunchKernelGGL(k_block_dots<T_IQ4_XS>, g, dim3(64), 0, st, w, xq, nb, isum, imin, d->iq4, d->signs); break;
  case T_IQ3_XXS: hipLaunchKernelGGL(k_block_dots<T_IQ3_XXS>, g, dim3(64), 0, st, w, xq, nb, isum, imin, d->iq3, d->signs); break;
  default: hipLaunchKernelGGL(k_block_dots<T_IQ2_XXS>, g, dim3(64), 0, st, w, xq, nb, isum, imin, d->grid, d->signs); break;
  }
  HIP_OK(hipGetLastError());
  HIP_OK(hipFreeAsync(xq, st));
  return 0;
}

// ---------------------------------------------------------------- routed layer

}  // extern "C"

namespace {
struct LayerWs {
  float *logits;
  int32_t *ids;
  float *weights;
  uint8_t *xq;
  int32_t *counts, *offs, *pairs, *active, *n_active;
  float *act;
  uint8_t *aq;
  float *y;
  float *act_s;
  uint8_t *aq_s;
  float *y_s;
  float *f_act;
  uint32_t *f_sync;
  int32_t *items, *n_items;    // MFMA work items of the gate/up launch
  int32_t *items2, *n_items2;  // and of the down launch when its tiling differs
};

size_t layer_ws(const zm_moe_layer *L, int S, uint8_t *base, LayerWs *w) {
  const int H = L->H, F = L->F, E = L->router.n_experts, K = L->router.topk, NS = L->n_slots;
  const int nbH = H / QK, nbF = F / QK;
  Bump b{base};
  LayerWs t{};
  t.logits = b.take<float>((size_t)S * E * 4);
  t.ids = b.take<int32_t>((size_t)S * K * 4);
  t.weights = b.take<float>((size_t)S * K * 4);
  t.xq = b.take<uint8_t>((size_t)S * q8_row_bytes(nbH));
  t.counts = b.take<int32_t>((size_t)NS * 4);
  t.offs = b.take<int32_t>((size_t)(NS + 1) * 4);
  t.pairs = b.take<int32_t>((size_t)S * K * 4);
  t.active = b.take<int32_t>((size_t)NS * 4);
  t.n_active = b.take<int32_t>(4);
  t.items = b.take<int32_t>((size_t)mmq_max_items(S * K, NS) * 4);
  t.n_items = b.take<int32_t>(4);
  t.items2 = b.take<int32_t>((size_t)mmq_max_items(S * K, NS) * 4);
  t.n_items2 = b.take<int32_t>(4);
  t.act = b.take<float>((size_t)S * K * F * 4);
  t.aq = b.take<uint8_t>((size_t)S * K * q8_row_bytes(nbF));
  t.y = b.take<float>((size_t)S * K * H * 4);
  if (L->F_shared > 0) {
    t.act_s = b.take<float>((size_t)S * L->F_shared * 4);
    t.aq_s = b.take<uint8_t>((size_t)S * q8_row_bytes(L->F_shared / QK));
    t.y_s = b.take<float>((size_t)S * H * 4);
  }
  // fused decode: act rows of every pair then the shared rows, their Q8_K
  // rows, and the sync words (zero at allocation, left at zero by every launch)
  const size_t fs = L->F_shared > 0 ? (size_t)L->F_shared : 0;
  t.f_act = b.take<float>(((size_t)S * K * F + S * fs) * 4);
  t.f_sync = b.take<uint32_t>((size_t)DEC_SYNC_WORDS * 4);
  if (w) *w = t;
  return b.off + 256;
}

int check_layer(const zm_moe_layer *L) {
  if (!L) return fail("null layer");
  if (L->H <= 0 || L->H % QK || L->H / QK > 64) return fail("H must be a multiple of 256, <= 16384");
  if (L->F <= 0 || L->F % QK || L->F / QK > 64) return fail("F must be a multiple of 256, <= 16384");
  if (!type_supported(L->type_gate) || L->type_up != L->type_gate || !type_supported(L->type_down))
    return fail("unsupported expert types (gate and up must share a type)");
  if (L->n_slots <= 0 || L->n_slots > BUCKET_MAX_E) return fail("n_slots out of range");
  if (L->router.n_experts <= 0 || L->router.n_experts > ROUTER_MAX_E) return fail("n_experts out of range");
  if (L->router.topk <= 0 || L->router.topk > 64 || L->router.topk > L->router.n_experts) return fail("bad topk");
  if (!L->route_map && L->n_slots != L->router.n_experts) return fail("n_slots != n_experts without a slot table");
  if (!L->w_gate || !L->w_up || !L->w_down) return fail("null expert weights");
  if (L->F_shared > 0) {
    if (L->F_shared % QK || L->F_shared / QK > 64 || !type_supported(L->type_shared) || !L->ws_gate || !L->ws_up ||
        !L->ws_down)
      return fail("bad shared expert");
  }
  if (L->router_w && L->H % 4) return fail("router GEMV needs H %% 4 == 0");
  return 0;
}
int units_per_block(int t) {
  return t == T_Q3_K || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K || t == T_IQ4_XS || t == T_IQ3_XXS ? 2 : 1;
}

DecFn find_decode(int tg, int td, int ts, int l1, int ir, int is) {
  if (DecFn f = find_decode_a(tg, td, ts, l1, ir, is)) return f;
  return find_decode_b(tg, td, ts, l1, ir, is);
}

bool fused_enabled() {
  const char *e = getenv("ZEROMOE_FUSED_DECODE");
  return !(e && e[0] == '0');
}

// grid of co-resident workgroups for a decode kernel (cached per device and kernel)
int decode_grid(DecFn fn, int *out) {
  static std::mutex mu;
  static struct Ent {
    int dev;
    DecFn fn;
    int grid;
  } cache[64];
  static int n = 0;
  int dev = 0;
  HIP_OK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(mu);
  for (int i = 0; i < n; ++i)
    if (cache[i].dev == dev && cache[i].fn == fn) {
      *out = cache[i].grid;
      return 0;
    }
  int per_cu = 0, cus = 0;
  HIP_OK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(fn), DEC_THREADS, 0));
  HIP_OK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const int grid = per_cu * cus;
  if (grid <= 0) return fail("decode kernel does not fit on a CU");
  if (n < 64) cache[n++] = Ent{dev, fn, grid};
  *out = grid;
  return 0;
}

// Returns 0 when launched, 1 when this shape takes the multi-kernel path, -1 on error.
int launch_fused(const zm_moe_layer *L, const float *x, const float *logits, int S, float *out, int32_t *ids,
                 float *wts, const LayerWs &w, const DeviceState *d, hipStream_t st) {
  const int H = L->H, F = L->F, E = L->router.n_experts, K = L->router.topk;
  const int nbH = H / QK, nbF = F / QK;
  const int Fs = L->F_shared > 0 ? L->F_shared : 0;
  const int nbFs = Fs / QK;
  if (!fused_enabled() || S > DEC_MAX_S || S * K > DEC_MAX_PAIRS || E > DEC_MAX_E)
    return 1;
  if (L->type_up != L->type_gate) return 1;
  const int u1 = nbH * units_per_block(L->type_gate);
  if (Fs && nbH * units_per_block(L->type_shared) > 64) return 1;
  // down rows: IQ2_XXS in half blocks (the decode kernel's H2)
  const int ir = (K * nbF * (L->type_down == T_IQ2_XXS ? 2 : units_per_block(L->type_down)) + 31) / 32;
  const int is = Fs ? (nbFs * units_per_block(L->type_shared) + 31) / 32 : 0;
  // lanes per routed gate/up row: 16 or 32, or 16 + 4 for rows of 20 units
  // where the kernel has that layout
  DecFn fn = nullptr;
  if (u1 == 20) fn = find_decode(L->type_gate, L->type_down, Fs ? L->type_shared : 0, 20, ir, is);
  if (!fn) {
    const int l1 = u1 <= 16 ? 16 : (u1 <= 32 ? 32 : 0);
    fn = find_decode(L->type_gate, L->type_down, Fs ? L->type_shared : 0, l1, ir, is);
  }
  if (!fn) return 1;
  int G = 0;
  if (decode_grid(fn, &G)) return -1;
  const long T1 = (long)S * K * F + (long)S * Fs;
  const size_t q8F = q8l_row_bytes(nbF), q8Fs = Fs ? q8l_row_bytes(nbFs) : 0;
  if ((size_t)S * q8l_row_bytes(nbH) > (size_t)DEC_LDS_Q8 || 2 * ((size_t)K * q8F + q8Fs) > (size_t)DEC_LDS_Q8) return 1;
  if (T1 >= (1l << 24) || (long)S * H >= (1l << 24)) return 1;  // float-reciprocal index math
  if ((T1 + QK - 1) / QK > DEC_MAX_ABLK) return 1;                // act block counters
  DecodeArgs a{};
  a.r = RouterArgs{logits, L->logit_bias, L->sel_bias, L->route_map, L->route_mask, E, K, L->router.gating,
                   L->router.n_groups, L->router.n_groups_used, L->router.weights_norm, L->router.weights_scale,
                   ids, wts};
  a.x = x;
  a.out = out;
  a.H = H;
  a.F = F;
  a.K = K;
  a.S = S;
  a.nbH = nbH;
  a.nbF = nbF;
  a.wg = (const uint8_t *)L->w_gate;
  a.wu = (const uint8_t *)L->w_up;
  a.wd = (const uint8_t *)L->w_down;
  a.g_rstride = row_bytes(L->type_gate, H);
  a.g_estride = a.g_rstride * F;
  a.d_rstride = row_bytes(L->type_down, F);
  a.d_estride = a.d_rstride * H;
  a.Fs = Fs;
  a.nbFs = nbFs;
  if (Fs) {
    a.sg = (const uint8_t *)L->ws_gate;
    a.su = (const uint8_t *)L->ws_up;
    a.sd = (const uint8_t *)L->ws_down;
    a.sg_rstride = row_bytes(L->type_shared, H);
    a.sd_rstride = row_bytes(L->type_shared, Fs);
  }
  {
    const size_t NSl = (size_t)L->n_slots;
    const size_t wgb = NSl * a.g_estride, wdb = NSl * a.d_estride;
    const size_t sgb = Fs ? (size_t)Fs * a.sg_rstride : 0, sdb = Fs ? (size_t)H * a.sd_rstride : 0;
    if (wgb >= (1ull << 31) || wdb >= (1ull << 31) || sgb >= (1ull << 31) || sdb >= (1ull << 31)) return 1;
    a.wg_bytes = (uint32_t)wgb;
    a.wd_bytes = (uint32_t)wdb;
    a.sg_bytes = (uint32_t)sgb;
    a.sd_bytes = (uint32_t)sdb;
  }
  a.act = w.f_act;
  a.sync = w.f_sync;
  auto uses = [&](int t) { return L->type_gate == t || L->type_down == t || (Fs && L->type_shared == t); };
  a.grid = uses(T_IQ4_XS) ? d->iq4 : (uses(T_IQ3_XXS) ? d->iq3 : d->grid);
  a.signs = d->signs;
  a.spin_limit = 1 << 23;
  // test hook: force the bounded waits to give up (a negative limit expires
  // every act-block wait on its first poll, whatever the counters show)
  if (const char *sl = getenv("ZEROMOE_SPIN_LIMIT"); sl && sl[0])
    a.spin_limit = atoi(sl);
  if (const char *tr = getenv("ZEROMOE_TRACE"); tr && tr[0] == '1') {
    DeviceState *dm = const_cast<DeviceState *>(d);
    if (dm->trace_n < (size_t)G * 8) {
      if (dm->trace) (void)hipFree(dm->trace);
      HIP_OK(hipMalloc(&dm->trace, (size_t)G * 8 * sizeof(uint64_t)));
      dm->trace_n = (size_t)G * 8;
    }
    HIP_OK(hipMemsetAsync(dm->trace, 0, dm->trace_n * sizeof(uint64_t), st));
    a.trace = dm->trace;
  }
  void *args[] = {&a};
  // A plain launch of exactly the co-resident grid: every workgroup is
  // dispatched at once on an otherwise idle device; the wait in the kernel is
  // bounded, so a device shared with other work degrades to an error status,
  // never a hang.  ZEROMOE_COOP=1 uses a cooperative launch instead.
  const char *coop = getenv("ZEROMOE_COOP");
  if (coop && coop[0] == '1')
    HIP_OK(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(fn), dim3(G), dim3(DEC_THREADS), args, 0, st));
  else
    HIP_OK(hipLaunchKernel(reinterpret_cast<const void *>(fn), dim3(G), dim3(DEC_THREADS), args, 0, st));
  return 0;
}

}  // namespace

extern "C" {

int zm_debug_trace(uint64_t *host, int n) {
  DeviceState *d;
  if (device_state(&d)) return -1;
  if (!d->trace) return 0;
  const int m = std::min<int>(n, (int)d->trace_n);
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(host, d->trace, (size_t)m * sizeof(uint64_t), hipMemcpyDeviceToHost));
  return m;
}

int zm_moe_status(const zm_moe_layer *layer, int S, void *workspace, void *stream) {
  if (check_layer(layer) || S <= 0 || !workspace) return -1;
  LayerWs w;
  layer_ws(layer, S, (uint8_t *)workspace, &w);
  uint32_t err = 0;
  HIP_OK(hipMemcpyAsync(&err, w.f_sync + 1, 4, hipMemcpyDeviceToHost, (hipStream_t)stream));
  HIP_OK(hipStreamSynchronize((hipStream_t)stream));
  if (err) {  // an expired wait leaves the arrival counters unknown: start them over
    HIP_OK(hipMemsetAsync(w.f_sync, 0, (size_t)DEC_SYNC_WORDS * 4, (hipStream_t)stream));
    HIP_OK(hipStreamSynchronize((hipStream_t)stream));
  }
  return (int)err;
}

size_t zm_moe_workspace_size(const zm_moe_layer *layer, int S) {
  if (check_layer(layer) || S <= 0) return 0;
  return layer_ws(layer, S, nullptr, nullptr);
}

int zm_moe_forward(const zm_moe_layer *L, const float *x, const float *logits, int S, float *out, int32_t *ids_out,
                   float *weights_out, void *workspace, size_t workspace_size, void *stream) {
  if (check_layer(L)) return -1;
  if (S <= 0 || !x || !out || (!logits && !L->router_w)) return fail("zm_moe_forward: bad arguments");
  if (S > 65535) return fail("S too large");
  if (!workspace || workspace_size < layer_ws(L, S, nullptr, nullptr)) return fail("workspace too small");
  DeviceState *d;
  if (device_state(&d)) return -1;
  hipStream_t st = (hipStream_t)stream;
  LayerWs w;
  layer_ws(L, S, (uint8_t *)workspace, &w);
  const int H = L->H, F = L->F, E = L->router.n_experts, K = L->router.topk, NS = L->n_slots;
  const int nbH = H / QK, nbF = F / QK;
  int32_t *ids = ids_out ? ids_out : w.ids;
  float *wts = weights_out ? weights_out : w.weights;

  // router
  const float *lg = logits;
  if (L->router_w) {
    // K slices so that ~512 workgroups stream the router weights; the partial
    // sums go through w.y (S*K*H floats, unused until the down projection)
    int KS = 1;
    while (KS < 16 && ((E + 15) / 16) * ((S + 15) / 16) * KS * 2 <= 512 && H % (64 * KS * 2) == 0 &&
           (size_t)KS * 2 * S * E <= (size_t)S * K * H)
      KS *= 2;
    if (S >= 8 && H % 64 == 0) {
      hipLaunchKernelGGL(k_router_gemm, dim3((E + 15) / 16, (S + 15) / 16, KS), dim3(256), 0, st, L->router_w, x, H,
                         E, S, w.y);
      hipLaunchKernelGGL(k_router_sum, dim3((S * E + 255) / 256), dim3(256), 0, st, w.y, S * E, KS, w.logits);
    } else
      hipLaunchKernelGGL(k_router_gemv, dim3(E), dim3(256), 0, st, L->router_w, x, H, E, S, w.logits);
    lg = w.logits;
  }
  {
    const int rc = launch_fused(L, x, lg, S, out, ids, wts, w, d, st);
    if (rc <= 0) return rc;
  }
  if (zm_router(&L->router, lg, L->logit_bias, L->sel_bias, L->route_map, L->route_mask, S, ids, wts, st))
    return -1;
  // activations -> Q8_K, buckets
  if (launch_quant(x, (size_t)H, nbH, S, w.xq, q8_row_bytes(nbH), 1, st)) return -1;
  // shared expert (dense over all tokens) on the side stream: it needs only
  // the Q8_K rows of x, and its gate/up, act quantization and down overlap
  // the router-dependent kernels; the combine waits for it
  auto launch_shared = [&](hipStream_t ss) -> int {
    const int Fs = L->F_shared, nbS = Fs / QK;
    GemvArgs c{};
    c.w0 = (const uint8_t *)L->ws_gate;
    c.w1 = (const uint8_t *)L->ws_up;
    c.w_rstride = row_bytes(L->type_shared, H);
    c.w_estride = 0;
    c.nrows = Fs;
    c.nb = nbH;
    c.xq = w.xq;
    c.xq_rstride = q8_row_bytes(nbH);
    c.xq_bytes = (uint32_t)((size_t)S * q8_row_bytes(nbH));
    c.ne11 = 1;
    c.K = 1;
    c.dense_S = S;
    c.out = w.act_s;
    c.out_s = Fs;
    c.out_k = 0;
    c.grid = d->grid;
    c.signs = d->signs;
    const int nps = S >= 4 ? 4 : (S >= 2 ? 2 : 1);
    {
      // 64-row tiles of the shared expert's F rows times (S / 32) items: a
      // one-wave workgroup per 16 rows when that leaves CUs idle
      const int cus = d->n_cu > 0 ? d->n_cu : 256;
      const int nw = (long)((Fs + 63) / 64) * ((S + 31) / 32) < cus ? 1 : 4;
      const int rc = launch_mmq(L->type_shared, true, c, (S + 31) / 32, (double)S, 2, ss, nw);
      if (rc < 0 || (rc > 0 && launch_gemv(L->type_shared, true, nps, c, 1, ss))) return -1;
    }
    if (launch_quant(w.act_s, (size_t)Fs, nbS, S, w.aq_s, q8_row_bytes(nbS), 1, ss)) return -1;
    GemvArgs e2 = c;
    e2.w0 = (const uint8_t *)L->ws_down;
    e2.w1 = nullptr;
    e2.w_rstride = row_bytes(L->type_shared, Fs);
    e2.nrows = H;
    e2.nb = nbS;
    e2.xq = w.aq_s;
    e2.xq_rstride = q8_row_bytes(nbS);
    e2.xq_bytes = (uint32_t)((size_t)S * q8_row_bytes(nbS));
    e2.out = w.y_s;
    e2.out_s = H;
    {
      const int rc = launch_mmq(L->type_shared, false, e2, (S + 31) / 32, (double)S, 2, ss);
      if (rc < 0 || (rc > 0 && launch_gemv(L->type_shared, false, nps, e2, 1, ss))) return -1;
    }
    return 0;
  };
  std::unique_lock<std::mutex> fork_lk;
  if (L->F_shared > 0) {
    fork_lk = std::unique_lock<std::mutex>(*d->fork_mu);
    HIP_OK(hipEventRecord(d->ev_fork, st));
    HIP_OK(hipStreamWaitEvent(d->side, d->ev_fork, 0));
    if (launch_shared(d->side)) return -1;
    HIP_OK(hipEventRecord(d->ev_join, d->side));
  }
  hipLaunchKernelGGL(k_bucket, dim3(1), dim3(1024), 0, st, ids, S * K, NS, w.counts, w.offs, w.pairs, w.active,
                     w.n_active);
  // gate/up + SwiGLU
  const int groups = std::min(NS, S * K);
  const int np = pick_np(S * K, NS);
  GemvArgs a{};
  a.w0 = (const uint8_t *)L->w_gate;
  a.w1 = (const uint8_t *)L->w_up;
  a.w_rstride = row_bytes(L->type_gate, H);
  a.w_estride = a.w_rstride * F;
  a.nrows = F;
  a.nb = nbH;
  a.xq = w.xq;
  a.xq_rstride = q8_row_bytes(nbH);
  a.ne11 = 1;
  a.K = K;
  a.n_active = w.n_active;
  a.active = w.active;
  a.offs = w.offs;
  a.pairs = w.pairs;
  a.out = w.act;
  a.out_s = (size_t)K * F;
  a.out_k = F;
  a.grid = d->grid;
  a.signs = d->signs;
  const double avg_pairs = (double)(S * K) / std::max(1, std::min(NS, S * K));
  // 16-token tiles per routed work item, per projection (mmq_tt); gate/up and
  // down take separate item lists when their tilings differ
  int tt_g = mmq_tt(L->type_gate, false), tt_d = mmq_tt(L->type_down, false);
  // items: at most one partial run per active expert plus the full runs
  auto max_items_for = [&](int tt) {
    return std::min(mmq_max_items(S * K, NS), (S * K + 16 * tt - 1) / (16 * tt) + std::min(NS, S * K));
  };
  auto cut_items = [&](int tt, int32_t *items, int32_t *n_items) {
    if (getenv_flag_off("ZEROMOE_MMQ_LPT") || NS > 1024)
      hipLaunchKernelGGL(k_mmq_items, dim3(1), dim3(1024), 0, st, w.n_active, w.active, w.offs, items, n_items,
                         16 * tt);
    else
      hipLaunchKernelGGL(k_mmq_items_lpt, dim3(1), dim3(1024), 0, st, w.n_active, w.active, w.offs, items, n_items,
                         16 * tt);
  };
  const bool mmq_g = mmq_applies(L->type_gate, avg_pairs), mmq_d = mmq_applies(L->type_down, avg_pairs);
  const bool split_items = mmq_g && mmq_d && tt_d != tt_g;
  if (!mmq_g && mmq_d) tt_g = tt_d;  // one list, cut for the down launch
  if (mmq_g || mmq_d) cut_items(tt_g, w.items, w.n_items);
  if (split_items) cut_items(tt_d, w.items2, w.n_items2);
  a.items = w.items;
  a.n_items = w.n_items;
  a.xq_bytes = (uint32_t)((size_t)S * q8_row_bytes(nbH));
  {
    const int rc = launch_mmq(L->type_gate, true, a, max_items_for(tt_g), avg_pairs, tt_g, st);
    if (rc < 0 || (rc > 0 && launch_gemv(L->type_gate, true, np, a, groups, st))) return -1;
  }
  // act -> Q8_K
  if (launch_quant(w.act, (size_t)F, nbF, S * K, w.aq, q8_row_bytes(nbF), 1, st)) return -1;
  // skipped routes (slot table -1) read as zero rows; router ids are always valid otherwise
  if (L->route_map)
    hipLaunchKernelGGL(k_fill_skipped, dim3((unsigned)std::min((H + 255) / 256, 64), (unsigned)std::min(S * K, 65535)), dim3(256), 0,
                     st, ids, (size_t)K, (size_t)1, K, S, NS, H, w.y, (size_t)K * H, (size_t)H);
  // down
  GemvArgs b = a;
  b.w0 = (const uint8_t *)L->w_down;
  b.w1 = nullptr;
  b.w_rstride = row_bytes(L->type_down, F);
  b.w_estride = b.w_rstride * H;
  b.nrows = H;
  b.nb = nbF;
  b.xq = w.aq;
  b.xq_rstride = q8_row_bytes(nbF);
  b.xq_bytes = (uint32_t)((size_t)S * K * q8_row_bytes(nbF));
  b.ne11 = K;
  b.out = w.y;
  b.out_s = (size_t)K * H;
  b.out_k = H;
  if (split_items) {
    b.items = w.items2;
    b.n_items = w.n_items2;
  } else {
    tt_d = tt_g;
  }
  {
    const int rc = launch_mmq(L->type_down, false, b, max_items_for(tt_d), avg_pairs, tt_d, st);
    if (rc < 0 || (rc > 0 && launch_gemv(L->type_down, false, np, b, groups, st))) return -1;
  }
  if (L->F_shared > 0) HIP_OK(hipStreamWaitEvent(st, d->ev_join, 0));  // the shared expert's y_s
  const float *ys = L->F_shared > 0 ? w.y_s : nullptr;
  if ((uintptr_t)out & 15)
    hipLaunchKernelGGL(k_combine1, dim3((H + 255) / 256, S), dim3(256), 0, st, w.y, wts, ys, H, K, out);
  else
    hipLaunchKernelGGL(k_combine, dim3((H + 1023) / 1024, S), dim3(256), 0, st, w.y, wts, ys, H, K, out);
  HIP_OK(hipGetLastError());
  return 0;
}

}  // extern "C"
