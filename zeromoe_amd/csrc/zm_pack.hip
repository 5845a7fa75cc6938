// zm_pack.hip -- expert-record unpack: device-local conversion from the
// transfer layout (one expert-major record [gate | up | down] per expert, so a
// routed expert crosses PCIe in one contiguous copy) into the three planar
// per-expert tensors MUL_MAT_ID reads.  Declared in include/zeromoe.h under the
// reference's symbol names (kernels/math/ggml_moe_pack.cu:127-179).
//
// Pure HBM streaming: each byte is read once and written once.  The grid is
// flat over (record, part, 16 KiB chunk); a workgroup copies one chunk with
// four 16-byte loads in flight per lane before its four stores.  Stores are
// non-temporal: the destination is not read again by this launch, and
// streaming it past the caches measured 6.9 TB/s against 5.4 TB/s for plain
// stores (and 5.3 TB/s for a device-to-device hipMemcpyAsync) on c2-sized
// records.  A part whose
// source and destination are both 16-byte aligned (every GGUF K-quant expert
// tensor is) takes the vector path; any other part is copied byte by byte.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../../include/zeromoe.h"
#include "zm_host.hpp"

using namespace zm;

namespace {

constexpr int PK_THREADS = 256;
constexpr int PK_UNROLL = 4;
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
constexpr size_t PK_CHUNK = (size_t)PK_THREADS * PK_UNROLL * 16;  // bytes per workgroup

struct UnpackArgs {
  const uint8_t *src;
  uint8_t *dst[3];        // gate, up, down bases
  size_t bytes[3];        // part sizes within one record
  size_t dst_stride[3];   // per-expert strides of the planar tensors
  size_t src_stride;      // record stride
  const int32_t *slots;   // compact record -> expert slot (NULL: record i -> expert i)
  uint32_t chunks;        // chunks per part (of the largest part)
};

__global__ __launch_bounds__(PK_THREADS) void k_moe_unpack(UnpackArgs a) {
  const uint32_t job = blockIdx.x / a.chunks;  // record * 3 + part
  const size_t off = (size_t)(blockIdx.x - job * a.chunks) * PK_CHUNK;
  const int rec = (int)(job / 3), part = (int)(job - 3u * (uint32_t)rec);
  const size_t nbytes = a.bytes[part];
  if (off >= nbytes) return;
  int slot = rec;
  if (a.slots) {
    slot = a.slots[rec];
    if (slot < 0) return;
  }
  size_t src_off = (size_t)rec * a.src_stride;
  if (part > 0) src_off += a.bytes[0];
  if (part > 1) src_off += a.bytes[1];
  const uint8_t *s = a.src + src_off + off;
  uint8_t *d = a.dst[part] + (size_t)slot * a.dst_stride[part] + off;
  const size_t n = nbytes - off < PK_CHUNK ? nbytes - off : PK_CHUNK;
  const int t = threadIdx.x;
  if ((((uintptr_t)s | (uintptr_t)d) & 15) == 0) {
    const size_t nv = n / 16;
    const v4u *sv = reinterpret_cast<const v4u *>(s);
    v4u *dv = reinterpret_cast<v4u *>(d);
    if (nv == (size_t)PK_THREADS * PK_UNROLL) {
      v4u r[PK_UNROLL];
#pragma unroll
      for (int u = 0; u < PK_UNROLL; ++u) r[u] = sv[u * PK_THREADS + t];
#pragma unroll
      for (int u = 0; u < PK_UNROLL; ++u) __builtin_nontemporal_store(r[u], dv + u * PK_THREADS + t);
      return;
    }
    for (size_t i = t; i < nv; i += PK_THREADS) __builtin_nontemporal_store(sv[i], dv + i);
    for (size_t i = nv * 16 + t; i < n; i += PK_THREADS) d[i] = s[i];
    return;
  }
  for (size_t i = t; i < n; i += PK_THREADS) d[i] = s[i];
}

int unpack(const void *src, void *gate, void *up, void *down, const int32_t *slots, bool scatter, int count,
           size_t src_stride, size_t gate_bytes, size_t up_bytes, size_t down_bytes, size_t gate_stride,
           size_t up_stride, size_t down_stride, hipStream_t st) {
  const char *who = scatter ? "launch_ggml_moe_unpack_scatter" : "launch_ggml_moe_unpack";
  if (!src || !gate || !up || !down || (scatter && !slots) || count <= 0) {
    fail("%s: null pointer or count <= 0", who);
    return hipErrorInvalidValue;
  }
  UnpackArgs a{};
  a.src = (const uint8_t *)src;
  a.dst[0] = (uint8_t *)gate;
  a.dst[1] = (uint8_t *)up;
  a.dst[2] = (uint8_t *)down;
  a.bytes[0] = gate_bytes;
  a.bytes[1] = up_bytes;
  a.bytes[2] = down_bytes;
  a.dst_stride[0] = gate_stride;
  a.dst_stride[1] = up_stride;
  a.dst_stride[2] = down_stride;
  a.src_stride = src_stride;
  a.slots = scatter ? slots : nullptr;
  size_t mx = gate_bytes > up_bytes ? gate_bytes : up_bytes;
  mx = mx > down_bytes ? mx : down_bytes;
  if (mx == 0) return hipSuccess;
  const size_t chunks = (mx + PK_CHUNK - 1) / PK_CHUNK;
  const size_t blocks = chunks * 3 * (size_t)count;
  if (blocks > 0x7fffffffull) {
    fail("%s: %d records of up to %zu bytes exceed one launch", who, count, mx);
    return hipErrorInvalidValue;
  }
  a.chunks = (uint32_t)chunks;
  hipLaunchKernelGGL(k_moe_unpack, dim3((unsigned)blocks), dim3(PK_THREADS), 0, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail("%s: %s", who, hipGetErrorString(e));
  return e;
}

}  // namespace

extern "C" {

int launch_ggml_moe_unpack(const void *src, void *gate, void *up, void *down, int count, size_t src_stride,
                           size_t gate_bytes, size_t up_bytes, size_t down_bytes, size_t gate_stride,
                           size_t up_stride, size_t down_stride, void *stream) {
  return unpack(src, gate, up, down, nullptr, false, count, src_stride, gate_bytes, up_bytes, down_bytes,
                gate_stride, up_stride, down_stride, (hipStream_t)stream);
}

int launch_ggml_moe_unpack_scatter(const void *src, void *gate, void *up, void *down, const int32_t *dst_slots,
                                   int count, size_t src_stride, size_t gate_bytes, size_t up_bytes,
                                   size_t down_bytes, size_t gate_stride, size_t up_stride, size_t down_stride,
                                   void *stream) {
  return unpack(src, gate, up, down, dst_slots, true, count, src_stride, gate_bytes, up_bytes, down_bytes,
                gate_stride, up_stride, down_stride, (hipStream_t)stream);
}

}  // extern "C"
