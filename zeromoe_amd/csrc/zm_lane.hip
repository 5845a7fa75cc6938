// zm_lane.hip -- the CPU lane of a hot/cold expert split: the layer's cold
// experts (held in host memory) run on the host cores while the GPU computes
// the hot ones, and the cold result is added to the GPU output.
//
// Reference: models/graph/early_ready_lane.hpp:75-211 (EarlyReadyLane: fork of
// activation, ids and router weights into private pinned buffers from inside
// the stream; the lane's CPU graph runs as soon as the fork event fires; the
// cold result is uploaded on a side stream and the merge waits on it), with the
// branch semantics of backends/ggml/moe_partial_route_ggml.hpp:21-60 (ids' =
// cold_map[ids], w' = w * cold_mask[ids]; out = hot + sum_topk(cold)) and
// models/graph/moe_block.hpp:160-185 (fork -> hot GPU work -> marker -> merge).
//
// The CPU computation is ggml's CPU MUL_MAT_ID layer: x quantized to Q8_K on
// one thread, gate/up rows of the token's cold routes split over the lane's
// threads, SwiGLU and the act's Q8_K on one thread, down rows split over the
// threads, then the k-ascending weighted sum of the cold routes.  The dots
// keep the integer grouping and float order of ggml's x86 kernels
// (bench/q2k_dot_bench.cpp:31-63, bench/q3k_q4k_dot_bench.cpp:73-125): per
// block, 8 int32 lane sums of 4 consecutive bytes of each 32-weight chunk, one
// fma per lane, the _mm256 horizontal-sum order at the end.  AVX-512 VNNI
// kernels are used where the host has them; the scalar kernels give the same
// bits.
#include <hip/hip_runtime.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

#include "../../include/zeromoe.h"
#include "zm_host.hpp"

namespace zm {
namespace cpu {

constexpr int QK = 256;

struct BlockQ2K {
  uint8_t scales[16];
  uint8_t qs[64];
  uint16_t d, dmin;
};
struct BlockQ3K {
  uint8_t hmask[32];
  uint8_t qs[64];
  uint8_t scales[12];
  uint16_t d;
};
struct BlockQ4K {
  uint16_t d, dmin;
  uint8_t scales[12];
  uint8_t qs[128];
};
struct BlockQ8K {
  float d;
  int8_t qs[256];
  int16_t bsums[16];
};
static_assert(sizeof(BlockQ2K) == 84 && sizeof(BlockQ3K) == 110 && sizeof(BlockQ4K) == 144 &&
                  sizeof(BlockQ8K) == 292,
              "ggml block layouts");

inline float f16(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// exp(x): Cody-Waite reduction by ln2 and a degree-7 Taylor polynomial, the
// operation sequence of the device exp_f32 (zm_device.hpp), so the lane's
// SwiGLU equals the GPU's bit for bit
inline float exp_f32(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __builtin_inff();
  if (x < -103.972084045410156f) return 0.0f;
  const float n = __builtin_rintf(x * 1.44269502162933349609375f);
  float r = __builtin_fmaf(n, -0.693145751953125f, x);
  r = __builtin_fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.98412701138295233249664306640625e-4f;
  p = __builtin_fmaf(p, r, 1.388888922519981861114501953125e-3f);
  p = __builtin_fmaf(p, r, 8.33333376795053482055664062500e-3f);
  p = __builtin_fmaf(p, r, 4.16666679084300994873046875000e-2f);
  p = __builtin_fmaf(p, r, 1.66666671633720397949218750000e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

// ggml quantize_row_q8_K: signed value of largest magnitude (first on ties),
// iscale = -127 / max, q = min(127, nearest_int(iscale * x)), 16-sums
void quantize_q8_K(const float *x, BlockQ8K *y, int n) {
  for (int i = 0; i < n / QK; ++i, x += QK) {
    float mx = 0.f, amax = 0.f;
    for (int j = 0; j < QK; ++j) {
      const float ax = __builtin_fabsf(x[j]);
      if (ax > amax) {
        amax = ax;
        mx = x[j];
      }
    }
    if (amax == 0.f) {
      std::memset(&y[i], 0, sizeof(BlockQ8K));
      continue;
    }
    const float iscale = -127.f / mx;
    for (int j = 0; j < QK; ++j) {
      const float v = iscale * x[j] + 12582912.f;  // round half to even (ggml nearest_int)
      int32_t b;
      std::memcpy(&b, &v, 4);
      const int q = (b & 0x007fffff) - 0x00400000;
      y[i].qs[j] = (int8_t)(q < 127 ? q : 127);
    }
    for (int j = 0; j < QK / 16; ++j) {
      int s = 0;
      for (int t = 0; t < 16; ++t) s += y[i].qs[16 * j + t];
      y[i].bsums[j] = (int16_t)s;
    }
    y[i].d = 1.f / iscale;
  }
}

// _mm256 horizontal-sum order: ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7))
inline float hsum8(const float a[8]) {
  const float r0 = a[4] + a[0], r1 = a[5] + a[1], r2 = a[6] + a[2], r3 = a[7] + a[3];
  return (r0 + r2) + (r1 + r3);
}

void q3_scales(const uint8_t *s12, int8_t *out) {
  uint32_t aux[4];
  std::memcpy(aux, s12, 12);
  const uint32_t m1 = 0x03030303u, m2 = 0x0f0f0f0fu, tmp = aux[2];
  aux[2] = ((aux[0] >> 4) & m2) | (((tmp >> 4) & m1) << 4);
  aux[3] = ((aux[1] >> 4) & m2) | (((tmp >> 6) & m1) << 4);
  aux[0] = (aux[0] & m2) | ((tmp & m1) << 4);
  aux[1] = (aux[1] & m2) | (((tmp >> 2) & m1) << 4);
  const uint8_t *b = reinterpret_cast<const uint8_t *>(aux);
  for (int i = 0; i < 16; ++i) out[i] = (int8_t)(b[i] - 32);
}

void q4_scale_min(const uint8_t *s, uint8_t sc[8], uint8_t m[8]) {
  for (int j = 0; j < 8; ++j) {
    if (j < 4) {
      sc[j] = s[j] & 63;
      m[j] = s[j + 4] & 63;
    } else {
      sc[j] = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
      m[j] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
  }
}

// ---------------------------------------------------------------- scalar dots

float dot_q2_K(int n, const BlockQ2K *x, const BlockQ8K *y) {
  float acc[8] = {0};
  for (int i = 0; i < n / QK; ++i) {
    const float d = y[i].d * f16(x[i].d);
    const float dmin = -y[i].d * f16(x[i].dmin);
    int32_t sumi[8] = {0};
    for (int l = 0; l < 8; ++l) {
      const int32_t prod =
          (x[i].scales[2 * l] >> 4) * y[i].bsums[2 * l] + (x[i].scales[2 * l + 1] >> 4) * y[i].bsums[2 * l + 1];
      acc[l] = __builtin_fmaf(dmin, (float)prod, acc[l]);
    }
    for (int j = 0; j < 2; ++j)
      for (int sh = 0; sh < 4; ++sh)
        for (int t = 0; t < 32; ++t) {
          const int q2 = (x[i].qs[32 * j + t] >> (2 * sh)) & 3;
          const int sc = x[i].scales[8 * j + 2 * sh + (t >= 16)] & 0xF;
          sumi[t >> 2] += sc * q2 * y[i].qs[128 * j + 32 * sh + t];
        }
    for (int l = 0; l < 8; ++l) acc[l] = __builtin_fmaf(d, (float)sumi[l], acc[l]);
  }
  return hsum8(acc);
}

float dot_q3_K(int n, const BlockQ3K *x, const BlockQ8K *y) {
  float acc[8] = {0};
  for (int i = 0; i < n / QK; ++i) {
    const float d = y[i].d * f16(x[i].d);
    int8_t sc[16];
    q3_scales(x[i].scales, sc);
    int32_t sumi[8] = {0};
    for (int j = 0; j < 2; ++j)
      for (int sh = 0; sh < 4; ++sh)
        for (int t = 0; t < 32; ++t) {
          const int q2 = (x[i].qs[32 * j + t] >> (2 * sh)) & 3;
          const int hb = (x[i].hmask[t] >> (4 * j + sh)) & 1;
          sumi[t >> 2] += sc[8 * j + 2 * sh + (t >= 16)] * (q2 - (hb ? 0 : 4)) * y[i].qs[128 * j + 32 * sh + t];
        }
    for (int l = 0; l < 8; ++l) acc[l] = __builtin_fmaf(d, (float)sumi[l], acc[l]);
  }
  return hsum8(acc);
}

float dot_q4_K(int n, const BlockQ4K *x, const BlockQ8K *y) {
  float acc[8] = {0}, accm[4] = {0};
  for (int i = 0; i < n / QK; ++i) {
    const float d = y[i].d * f16(x[i].d);
    const float dmin = -y[i].d * f16(x[i].dmin);
    uint8_t sc[8], m[8];
    q4_scale_min(x[i].scales, sc, m);
    int32_t s32[8];
    for (int j = 0; j < 8; ++j) s32[j] = y[i].bsums[2 * j] + y[i].bsums[2 * j + 1];
    for (int l = 0; l < 4; ++l)
      accm[l] = __builtin_fmaf(dmin, (float)(m[2 * l] * s32[2 * l] + m[2 * l + 1] * s32[2 * l + 1]), accm[l]);
    int32_t sumi[8] = {0};
    for (int j = 0; j < 4; ++j)
      for (int t = 0; t < 32; ++t) {
        const uint8_t b = x[i].qs[32 * j + t];
        sumi[t >> 2] += sc[2 * j] * (b & 0xF) * y[i].qs[64 * j + t];
        sumi[t >> 2] += sc[2 * j + 1] * (b >> 4) * y[i].qs[64 * j + 32 + t];
      }
    for (int l = 0; l < 8; ++l) acc[l] = __builtin_fmaf(d, (float)sumi[l], acc[l]);
  }
  return hsum8(acc) + ((accm[0] + accm[2]) + (accm[1] + accm[3]));
}

// ---------------------------------------------------------------- AVX-512 VNNI dots
#if defined(__x86_64__)
#define ZM_AVX512 __attribute__((target("avx512f,avx512bw,avx512vl,avx512vnni,avx512dq,fma")))

// int32 lane l of a 64-byte chunk pair k -> its 16-weight sub-block 4k + (l >> 2)
ZM_AVX512 inline __m512i lanes_of_4(int base) {
  return _mm512_setr_epi32(base, base, base, base, base + 1, base + 1, base + 1, base + 1, base + 2, base + 2,
                           base + 2, base + 2, base + 3, base + 3, base + 3, base + 3);
}
// per 16-bit word shift: s0 in the low 32 bytes, s1 in the high 32
ZM_AVX512 inline __m512i shifts(int s0, int s1) {
  return _mm512_inserti64x4(_mm512_castsi256_si512(_mm256_set1_epi16((short)s0)), _mm256_set1_epi16((short)s1), 1);
}
ZM_AVX512 inline float finish(__m256 acc) {
  float a[8];
  _mm256_storeu_ps(a, acc);
  return hsum8(a);
}
// the 16 int32 lanes folded to the 8 lane classes (byte group t >> 2 of a 32-byte chunk)
ZM_AVX512 inline __m256i fold16(__m512i v) {
  return _mm256_add_epi32(_mm512_castsi512_si256(v), _mm512_extracti64x4_epi64(v, 1));
}

ZM_AVX512 float dot_q2_K_avx512(int n, const BlockQ2K *x, const BlockQ8K *y) {
  const __m512i m3 = _mm512_set1_epi8(3);
  const __m512i sh[2] = {shifts(0, 2), shifts(4, 6)};
  __m256 acc = _mm256_setzero_ps();
  for (int i = 0; i < n / QK; ++i) {
    const float d = y[i].d * f16(x[i].d);
    const float dmin = -y[i].d * f16(x[i].dmin);
    const __m128i sc8 = _mm_loadu_si128(reinterpret_cast<const __m128i *>(x[i].scales));
    const __m256i m16 = _mm256_cvtepu8_epi16(_mm_and_si128(_mm_srli_epi16(sc8, 4), _mm_set1_epi8(0x0F)));
    const __m256i prod = _mm256_madd_epi16(m16, _mm256_loadu_si256(reinterpret_cast<const __m256i *>(y[i].bsums)));
    acc = _mm256_fmadd_ps(_mm256_set1_ps(dmin), _mm256_cvtepi32_ps(prod), acc);
    const __m512i sc32 = _mm512_and_si512(_mm512_cvtepu8_epi32(sc8), _mm512_set1_epi32(0xF));
    __m512i sumi = _mm512_setzero_si512();
    for (int j = 0; j < 2; ++j) {
      const __m512i q = _mm512_broadcast_i64x4(_mm256_loadu_si256(reinterpret_cast<const __m256i *>(x[i].qs + 32 * j)));
      for (int h = 0; h < 2; ++h) {
        const int k = 2 * j + h;
        const __m512i w = _mm512_and_si512(_mm512_srlv_epi16(q, sh[h]), m3);
        const __m512i dp = _mm512_dpbusd_epi32(_mm512_setzero_si512(), w, _mm512_loadu_si512(y[i].qs + 64 * k));
        sumi = _mm512_add_epi32(sumi, _mm512_mullo_epi32(dp, _mm512_permutexvar_epi32(lanes_of_4(4 * k), sc32)));
      }
    }
    acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(fold16(sumi)), acc);
  }
  return finish(acc);
}

ZM_AVX512 float dot_q3_K_avx512(int n, const BlockQ3K *x, const BlockQ8K *y) {
  const __m512i m3 = _mm512_set1_epi8(3), m1 = _mm512_set1_epi8(1);
  const __m512i sh[2] = {shifts(0, 2), shifts(4, 6)};
  __m256 acc = _mm256_setzero_ps();
  for (int i = 0; i < n / QK; ++i) {
    const float d = y[i].d * f16(x[i].d);
    int8_t sc[16];
    q3_scales(x[i].scales, sc);
    const __m512i sc32 = _mm512_cvtepi8_epi32(_mm_loadu_si128(reinterpret_cast<const __m128i *>(sc)));
    // 4 * (high bit clear): bit 2k (low half) / 2k + 1 (high half) of hmask[t]
    const __m512i nh = _mm512_broadcast_i64x4(_mm256_xor_si256(
        _mm256_loadu_si256(reinterpret_cast<const __m256i *>(x[i].hmask)), _mm256_set1_epi8(-1)));
    __m512i sumi = _mm512_setzero_si512();
    for (int j = 0; j < 2; ++j) {
      const __m512i q = _mm512_broadcast_i64x4(_mm256_loadu_si256(reinterpret_cast<const __m256i *>(x[i].qs + 32 * j)));
      for (int h = 0; h < 2; ++h) {
        const int k = 2 * j + h;
        const __m512i w = _mm512_and_si512(_mm512_srlv_epi16(q, sh[h]), m3);
        const __m512i n4 = _mm512_slli_epi16(_mm512_and_si512(_mm512_srlv_epi16(nh, shifts(2 * k, 2 * k + 1)), m1), 2);
        const __m512i q8 = _mm512_loadu_si512(y[i].qs + 64 * k);
        const __m512i dp = _mm512_sub_epi32(_mm512_dpbusd_epi32(_mm512_setzero_si512(), w, q8),
                                            _mm512_dpbusd_epi32(_mm512_setzero_si512(), n4, q8));
        sumi = _mm512_add_epi32(sumi, _mm512_mullo_epi32(dp, _mm512_permutexvar_epi32(lanes_of_4(4 * k), sc32)));
      }
    }
    acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(fold16(sumi)), acc);
  }
  return finish(acc);
}

ZM_AVX512 float dot_q4_K_avx512(int n, const BlockQ4K *x, const BlockQ8K *y) {
  const __m512i m15 = _mm512_set1_epi8(0x0F);
  const __m512i nib = shifts(0, 4);  // low nibbles against the chunk's first 32 q8, high against the second
  __m256 acc = _mm256_setzero_ps();
  __m128 accm = _mm_setzero_ps();
  for (int i = 0; i < n / QK; ++i) {
    const float d = y[i].d * f16(x[i].d);
    const float dmin = -y[i].d * f16(x[i].dmin);
    uint8_t sc[8], m[8];
    q4_scale_min(x[i].scales, sc, m);
    // mins: lane l = m[2l] * s32[2l] + m[2l+1] * s32[2l+1], s32 = 32-weight bsums
    const __m128i bs = _mm_hadd_epi16(_mm_loadu_si128(reinterpret_cast<const __m128i *>(y[i].bsums)),
                                      _mm_loadu_si128(reinterpret_cast<const __m128i *>(y[i].bsums + 8)));
    int16_t mm[8];
    for (int j = 0; j < 8; ++j) mm[j] = m[j];
    const __m128i prod = _mm_madd_epi16(_mm_loadu_si128(reinterpret_cast<const __m128i *>(mm)), bs);
    accm = _mm_fmadd_ps(_mm_set1_ps(dmin), _mm_cvtepi32_ps(prod), accm);
    __m512i sumi = _mm512_setzero_si512();
    for (int j = 0; j < 4; ++j) {
      const __m512i q = _mm512_broadcast_i64x4(_mm256_loadu_si256(reinterpret_cast<const __m256i *>(x[i].qs + 32 * j)));
      const __m512i w = _mm512_and_si512(_mm512_srlv_epi16(q, nib), m15);
      const __m512i dp = _mm512_dpbusd_epi32(_mm512_setzero_si512(), w, _mm512_loadu_si512(y[i].qs + 64 * j));
      const __m512i s = _mm512_inserti64x4(_mm512_set1_epi32(sc[2 * j]), _mm256_set1_epi32(sc[2 * j + 1]), 1);
      sumi = _mm512_add_epi32(sumi, _mm512_mullo_epi32(dp, s));
    }
    acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(fold16(sumi)), acc);
  }
  float am[4];
  _mm_storeu_ps(am, accm);
  return finish(acc) + ((am[0] + am[2]) + (am[1] + am[3]));
}

bool host_has_avx512() {
  return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
         __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512vnni") &&
         __builtin_cpu_supports("avx512dq");
}
#else
bool host_has_avx512() { return false; }
#endif

using DotFn = float (*)(int, const void *, const BlockQ8K *);

DotFn pick_dot(int type, bool vec) {
#if defined(__x86_64__)
  if (vec) {
    if (type == ZM_TYPE_Q2_K) return [](int n, const void *w, const BlockQ8K *y) {
      return dot_q2_K_avx512(n, static_cast<const BlockQ2K *>(w), y);
    };
    if (type == ZM_TYPE_Q3_K) return [](int n, const void *w, const BlockQ8K *y) {
      return dot_q3_K_avx512(n, static_cast<const BlockQ3K *>(w), y);
    };
    if (type == ZM_TYPE_Q4_K) return [](int n, const void *w, const BlockQ8K *y) {
      return dot_q4_K_avx512(n, static_cast<const BlockQ4K *>(w), y);
    };
  }
#endif
  if (type == ZM_TYPE_Q2_K)
    return [](int n, const void *w, const BlockQ8K *y) { return dot_q2_K(n, static_cast<const BlockQ2K *>(w), y); };
  if (type == ZM_TYPE_Q3_K)
    return [](int n, const void *w, const BlockQ8K *y) { return dot_q3_K(n, static_cast<const BlockQ3K *>(w), y); };
  if (type == ZM_TYPE_Q4_K)
    return [](int n, const void *w, const BlockQ8K *y) { return dot_q4_K(n, static_cast<const BlockQ4K *>(w), y); };
  return nullptr;
}

size_t row_bytes(int type, int n) {
  const int bb = type == ZM_TYPE_Q2_K ? 84 : (type == ZM_TYPE_Q3_K ? 110 : 144);
  return (size_t)(n / QK) * bb;
}

// ---------------------------------------------------------------- a small fork-join pool

// n_threads - 1 workers plus the calling thread run fn(i) for i in [0, n),
// chunks taken from a shared counter; run() returns when all are done.
class Pool {
 public:
  explicit Pool(int n_threads) {
    for (int t = 1; t < n_threads; ++t) workers_.emplace_back([this] { loop(); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
      ++gen_;
    }
    cv_.notify_all();
    for (auto &w : workers_) w.join();
  }
  void run(int n, int chunk, const std::function<void(int, int)> &fn) {
    {
      std::lock_guard<std::mutex> lk(mu_);
      fn_ = &fn;
      n_ = n;
      chunk_ = chunk;
      next_.store(0);
      busy_ = (int)workers_.size();
      ++gen_;
    }
    cv_.notify_all();
    work();
    std::unique_lock<std::mutex> lk(mu_);
    done_cv_.wait(lk, [this] { return busy_ == 0; });
    fn_ = nullptr;
  }

 private:
  void work() {
    for (;;) {
      const int b = next_.fetch_add(chunk_);
      if (b >= n_) break;
      (*fn_)(b, std::min(n_, b + chunk_));
    }
  }
  void loop() {
    uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return gen_ != seen; });
        seen = gen_;
        if (stop_) return;
      }
      work();
      {
        std::lock_guard<std::mutex> lk(mu_);
        if (--busy_ == 0) done_cv_.notify_all();
      }
    }
  }
  std::vector<std::thread> workers_;
  std::mutex mu_;
  std::condition_variable cv_, done_cv_;
  const std::function<void(int, int)> *fn_ = nullptr;
  std::atomic<int> next_{0};
  int n_ = 0, chunk_ = 1, busy_ = 0;
  uint64_t gen_ = 0;
  bool stop_ = false;
};

}  // namespace cpu

namespace {

__global__ void k_lane_add(float *__restrict__ out, const float *__restrict__ cold, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = out[i] + cold[i];
}

int64_t now_ns() {
  return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

}  // namespace
}  // namespace zm

using namespace zm;

struct zm_cold_lane {
  zm_cold_lane_desc d{};
  std::vector<int32_t> map;
  std::vector<float> mask;
  cpu::DotFn dot_g = nullptr, dot_u = nullptr, dot_d = nullptr;
  size_t rg = 0, ru = 0, rd = 0;
  bool vec = false;
  std::unique_ptr<cpu::Pool> pool;
  // per-call scratch (sized for max_tokens at creation)
  std::vector<cpu::BlockQ8K> xq, aq;
  std::vector<float> g, u, a, y;
  // device side, set up on the first fork
  bool hip_ready = false;
  int device = -1;
  float *h_x = nullptr, *h_w = nullptr, *h_out = nullptr;
  int32_t *h_ids = nullptr;
  float *d_cold = nullptr;
  // forked: the fork's copies landed; uploaded: a merge's upload of h_out
  // finished (h_out may be rewritten); added: a merge's add finished (d_cold
  // may be rewritten)
  hipEvent_t forked = nullptr, uploaded = nullptr, added = nullptr;
  bool merged_once = false;
  int forked_S = 0;
  hipStream_t side = nullptr;
  // the lane thread
  std::thread worker;
  std::mutex mu;
  std::condition_variable cv;
  int pending_S = 0;       // > 0: a forked call waits for the worker
  bool result_ready = false, stop = false;
  int status = 0;
  zm_cold_lane_stats stats{};

  // out[s] = sum over cold routes k (ascending) of w'_k * y_k: the cold branch of
  // the layer for S tokens, all on the host
  void compute(const float *x, const int32_t *ids, const float *w, int S, float *out) {
    const int H = d.H, F = d.F, K = d.topk, nbF = F / cpu::QK;
    for (int s = 0; s < S; ++s) {
      cpu::quantize_q8_K(x + (size_t)s * H, xq.data(), H);
      int slot[64];
      float wk[64];
      int nr = 0;
      for (int k = 0; k < K; ++k) {
        const int e = ids[(size_t)s * K + k];
        if (e < 0 || e >= d.n_experts) continue;
        const int sl = map[e];
        if (sl < 0) continue;
        slot[nr] = sl;
        wk[nr] = w[(size_t)s * K + k] * (mask.empty() ? 1.0f : mask[e]);
        ++nr;
      }
      float *o = out + (size_t)s * H;
      if (nr == 0) {
        std::memset(o, 0, sizeof(float) * (size_t)H);
        continue;
      }
      const uint8_t *wg = static_cast<const uint8_t *>(d.w_gate), *wu = static_cast<const uint8_t *>(d.w_up),
                    *wd = static_cast<const uint8_t *>(d.w_down);
      const size_t eg = rg * (size_t)F, eu = ru * (size_t)F, ed = rd * (size_t)H;
      pool->run(nr * F, 16, [&](int b, int e) {
        for (int r = b; r < e; ++r) {
          const int j = r / F, n = r % F;
          g[r] = dot_g(H, wg + (size_t)slot[j] * eg + (size_t)n * rg, xq.data());
          u[r] = dot_u(H, wu + (size_t)slot[j] * eu + (size_t)n * ru, xq.data());
        }
      });
      for (int j = 0; j < nr; ++j) {
        for (int n = 0; n < F; ++n) {
          const float gv = g[(size_t)j * F + n];
          a[(size_t)j * F + n] = gv / (1.0f + cpu::exp_f32(-gv)) * u[(size_t)j * F + n];
        }
        cpu::quantize_q8_K(a.data() + (size_t)j * F, aq.data() + (size_t)j * nbF, F);
      }
      pool->run(nr * H, 64, [&](int b, int e) {
        for (int r = b; r < e; ++r) {
          const int j = r / H, h = r % H;
          y[r] = dot_d(F, wd + (size_t)slot[j] * ed + (size_t)h * rd, aq.data() + (size_t)j * nbF);
        }
      });
      // ggml_mul(down, weights) then sum_topk in k order; skipped routes add 0
      for (int h = 0; h < H; ++h) {
        float acc = wk[0] * y[h];
        for (int j = 1; j < nr; ++j) acc = acc + wk[j] * y[(size_t)j * H + h];
        o[h] = acc;
      }
    }
  }

  void loop() {
    for (;;) {
      int S;
      {
        std::unique_lock<std::mutex> lk(mu);
        cv.wait(lk, [&] { return pending_S > 0 || stop; });
        if (stop) return;
        S = pending_S;
      }
      int st = 0;
      if (hipEventSynchronize(forked) != hipSuccess) st = -1;
      // the previous merge's upload still reads h_out until its event completes
      if (merged_once && hipEventSynchronize(uploaded) != hipSuccess) st = -1;
      stats.compute_begin_ns = now_ns();
      if (!st) compute(h_x, h_ids, h_w, S, h_out);
      stats.compute_end_ns = now_ns();
      {
        std::lock_guard<std::mutex> lk(mu);
        status = st;
        pending_S = 0;
        result_ready = true;
      }
      cv.notify_all();
    }
  }

  int setup_hip() {
    if (hip_ready) return 0;
    HIP_OK(hipGetDevice(&device));
    const size_t T = (size_t)d.max_tokens;
    HIP_OK(hipHostMalloc((void **)&h_x, T * d.H * sizeof(float), hipHostMallocDefault));
    HIP_OK(hipHostMalloc((void **)&h_out, T * d.H * sizeof(float), hipHostMallocDefault));
    HIP_OK(hipHostMalloc((void **)&h_w, T * d.topk * sizeof(float), hipHostMallocDefault));
    HIP_OK(hipHostMalloc((void **)&h_ids, T * d.topk * sizeof(int32_t), hipHostMallocDefault));
    HIP_OK(hipMalloc((void **)&d_cold, T * d.H * sizeof(float)));
    HIP_OK(hipEventCreateWithFlags(&forked, hipEventDisableTiming));
    HIP_OK(hipEventCreateWithFlags(&uploaded, hipEventDisableTiming));
    HIP_OK(hipEventCreateWithFlags(&added, hipEventDisableTiming));
    HIP_OK(hipStreamCreateWithFlags(&side, hipStreamNonBlocking));
    worker = std::thread([this] { loop(); });
    hip_ready = true;
    return 0;
  }

  ~zm_cold_lane() {
    if (worker.joinable()) {
      {
        std::lock_guard<std::mutex> lk(mu);
        stop = true;
      }
      cv.notify_all();
      worker.join();
    }
    if (hip_ready) {
      (void)hipSetDevice(device);
      (void)hipStreamSynchronize(side);
      (void)hipStreamDestroy(side);
      (void)hipEventDestroy(forked);
      (void)hipEventDestroy(uploaded);
      (void)hipEventDestroy(added);
      (void)hipFree(d_cold);
      (void)hipHostFree(h_x);
      (void)hipHostFree(h_out);
      (void)hipHostFree(h_w);
      (void)hipHostFree(h_ids);
    }
  }
};

extern "C" {

zm_cold_lane *zm_cold_lane_create(const zm_cold_lane_desc *d) {
  if (!d || d->H <= 0 || d->H % 256 || d->F <= 0 || d->F % 256 || d->topk <= 0 || d->topk > 64 ||
      d->n_experts <= 0 || d->n_slots <= 0 || d->max_tokens <= 0 || !d->route_map || !d->w_gate || !d->w_up ||
      !d->w_down) {
    fail("zm_cold_lane_create: bad descriptor");
    return nullptr;
  }
  const bool vec = cpu::host_has_avx512() && !d->scalar;
  cpu::DotFn dg = cpu::pick_dot(d->type_gate, vec), du = cpu::pick_dot(d->type_up, vec),
             dd = cpu::pick_dot(d->type_down, vec);
  if (!dg || !du || !dd) {
    fail("zm_cold_lane_create: the CPU lane supports Q2_K, Q3_K and Q4_K experts");
    return nullptr;
  }
  auto *L = new zm_cold_lane();
  L->d = *d;
  L->vec = vec;
  L->map.assign(d->route_map, d->route_map + d->n_experts);
  for (int32_t &v : L->map)
    if (v >= d->n_slots) v = -1;  // slots beyond the host pool are not owned
  if (d->route_mask) L->mask.assign(d->route_mask, d->route_mask + d->n_experts);
  L->dot_g = dg;
  L->dot_u = du;
  L->dot_d = dd;
  L->rg = cpu::row_bytes(d->type_gate, d->H);
  L->ru = cpu::row_bytes(d->type_up, d->H);
  L->rd = cpu::row_bytes(d->type_down, d->F);
  const int K = d->topk;
  L->xq.resize(d->H / cpu::QK);
  L->aq.resize((size_t)K * (d->F / cpu::QK));
  L->g.resize((size_t)K * d->F);
  L->u.resize((size_t)K * d->F);
  L->a.resize((size_t)K * d->F);
  L->y.resize((size_t)K * d->H);
  L->pool.reset(new cpu::Pool(d->n_threads > 0 ? d->n_threads : 1));
  L->stats.vectorized = vec ? 1 : 0;
  return L;
}

void zm_cold_lane_destroy(zm_cold_lane *lane) { delete lane; }

int zm_cold_lane_compute_host(zm_cold_lane *L, const float *x, const int32_t *ids, const float *weights, int S,
                              float *out) {
  if (!L || !x || !ids || !weights || !out || S <= 0 || S > L->d.max_tokens)
    return fail("zm_cold_lane_compute_host: bad arguments");
  std::lock_guard<std::mutex> lk(L->mu);
  if (L->pending_S > 0) return fail("zm_cold_lane_compute_host: a forked call is in flight");
  L->compute(x, ids, weights, S, out);
  return 0;
}

int zm_cold_lane_fork(zm_cold_lane *L, const float *x, const int32_t *ids, const float *weights, int S,
                      void *stream) {
  if (!L || !x || !ids || !weights || S <= 0 || S > L->d.max_tokens) return fail("zm_cold_lane_fork: bad arguments");
  if (L->setup_hip()) return -1;
  {
    std::lock_guard<std::mutex> lk(L->mu);
    if (L->pending_S > 0 || L->result_ready) return fail("zm_cold_lane_fork: the previous call was not merged");
  }
  hipStream_t st = (hipStream_t)stream;
  const size_t K = (size_t)L->d.topk;
  HIP_OK(hipMemcpyAsync(L->h_x, x, (size_t)S * L->d.H * sizeof(float), hipMemcpyDeviceToHost, st));
  HIP_OK(hipMemcpyAsync(L->h_ids, ids, (size_t)S * K * sizeof(int32_t), hipMemcpyDeviceToHost, st));
  HIP_OK(hipMemcpyAsync(L->h_w, weights, (size_t)S * K * sizeof(float), hipMemcpyDeviceToHost, st));
  HIP_OK(hipEventRecord(L->forked, st));
  L->stats.fork_ns = now_ns();
  {
    std::lock_guard<std::mutex> lk(L->mu);
    L->pending_S = S;
    L->forked_S = S;
  }
  L->cv.notify_all();
  return 0;
}

int zm_cold_lane_merge(zm_cold_lane *L, float *out, int S, void *stream) {
  if (!L || !out || S <= 0 || S > L->d.max_tokens || !L->hip_ready) return fail("zm_cold_lane_merge: bad arguments");
  int st_code;
  {
    std::unique_lock<std::mutex> lk(L->mu);
    if (L->pending_S == 0 && !L->result_ready) return fail("zm_cold_lane_merge: nothing forked");
    L->cv.wait(lk, [&] { return L->result_ready; });
    L->result_ready = false;
    st_code = L->status;
  }
  L->stats.merge_ns = now_ns();
  if (st_code) return fail("zm_cold_lane_merge: the fork's copies failed");
  if (S != L->forked_S) return fail("zm_cold_lane_merge: S differs from the forked call's");
  hipStream_t st = (hipStream_t)stream;
  // upload on the lane's side stream, then the caller's stream waits and adds;
  // the upload first waits for the previous merge's add, which read d_cold on
  // the caller's stream of that call
  const size_t n = (size_t)S * L->d.H;
  if (L->merged_once) HIP_OK(hipStreamWaitEvent(L->side, L->added, 0));
  HIP_OK(hipMemcpyAsync(L->d_cold, L->h_out, n * sizeof(float), hipMemcpyHostToDevice, L->side));
  HIP_OK(hipEventRecord(L->uploaded, L->side));
  HIP_OK(hipStreamWaitEvent(st, L->uploaded, 0));
  hipLaunchKernelGGL(k_lane_add, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, L->d_cold, (int)n);
  HIP_OK(hipGetLastError());
  HIP_OK(hipEventRecord(L->added, st));
  L->merged_once = true;
  return 0;
}

int zm_cold_lane_get_stats(const zm_cold_lane *L, zm_cold_lane_stats *s) {
  if (!L || !s) return fail("zm_cold_lane_get_stats: null argument");
  *s = L->stats;
  return 0;
}

}  // extern "C"
