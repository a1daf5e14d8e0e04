// Host-to-device row gather of bf16 K / V (the reference's UVA gather,
// Z/cache_hub/gather_trans/trans_h2d.cu:43-188 / trans_h2d.py:65-166): the
// kernel reads rows of pinned host memory through their device alias and
// writes them to HBM, so only the selected rows cross the host link.
//
//   dense:  dst[b, h, slot, :] = src[b, h, idx[b, h, slot], :],  slot < topk
//   packed: for segment vh = b * kv_heads + h, slot < cu_topk[vh+1] - cu_topk[vh]:
//           dst[cu_k[vh] + sl_end + slot, :] = src[b, h, idx[cu_topk[vh] + slot], :]
//           (rows [cu_k[vh], cu_k[vh] + sl_end) are the caller's sink + local)
//
// Rows are 256 B (head_dim 128).  Sixteen lanes move one row as 16-byte
// words; a 256-thread block moves 16 rows of K (blockIdx.z == 0) or V.
// An index outside [0, src_len) (or a packed destination outside the buffer)
// leaves its destination row untouched: the reference reads whatever address
// it yields, which in host memory would fault the device.
#include "zkv_common.hpp"

namespace zkv {
namespace {

constexpr int kRowWords = 16;  // 16-byte words per 128-dim bf16 row

__global__ __launch_bounds__(256) void h2d_gather_kernel(
    const u32x4_t* __restrict__ src_k, const u32x4_t* __restrict__ src_v, int src_len,
    const int64_t* __restrict__ idx, int topk, u32x4_t* __restrict__ dst_k, u32x4_t* __restrict__ dst_v,
    int dst_len, int64_t n_rows) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  if (r >= n_rows) return;
  const int w = threadIdx.x & 15;
  const int64_t bh = r / topk;
  const int slot = static_cast<int>(r - bh * topk);
  const int64_t index = idx[r];
  if (index < 0 || index >= src_len) return;
  const u32x4_t* src = blockIdx.z == 0 ? src_k : src_v;
  u32x4_t* dst = blockIdx.z == 0 ? dst_k : dst_v;
  dst[(bh * dst_len + slot) * kRowWords + w] = src[(bh * src_len + index) * kRowWords + w];
}

__global__ __launch_bounds__(256) void h2d_gather_packed_kernel(
    const u32x4_t* __restrict__ src_k, const u32x4_t* __restrict__ src_v, int kv_heads, int src_len,
    u32x4_t* __restrict__ dst_k, u32x4_t* __restrict__ dst_v, int64_t total_k,
    const int64_t* __restrict__ idx, int64_t total_topk, const int32_t* __restrict__ cu_topk,
    const int32_t* __restrict__ cu_k, int sl_end) {
  const int vh = blockIdx.x;
  const int slot = blockIdx.y * 16 + (threadIdx.x >> 4);
  const int w = threadIdx.x & 15;
  const int seg_start = cu_topk[vh];
  const int seg_len = cu_topk[vh + 1] - seg_start;
  if (slot >= seg_len) return;
  const int64_t pos = static_cast<int64_t>(seg_start) + slot;
  if (pos < 0 || pos >= total_topk) return;
  const int64_t index = idx[pos];
  const int64_t dst_row = static_cast<int64_t>(cu_k[vh]) + sl_end + slot;
  if (index < 0 || index >= src_len || dst_row < 0 || dst_row >= total_k) return;
  const int b = vh / kv_heads, h = vh - b * kv_heads;
  const int64_t src_row = (static_cast<int64_t>(b) * kv_heads + h) * src_len + index;
  const u32x4_t* src = blockIdx.z == 0 ? src_k : src_v;
  u32x4_t* dst = blockIdx.z == 0 ? dst_k : dst_v;
  dst[dst_row * kRowWords + w] = src[src_row * kRowWords + w];
}

// Device alias of a pinned host buffer (hipHostGetDevicePointer), or an error.
int device_alias(const void* host, const char* name, const u32x4_t** out) {
  void* d = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&d, const_cast<void*>(host), 0);
  if (e != hipSuccess || d == nullptr) {
    (void)hipGetLastError();  // the failed lookup must not surface at the caller's next HIP call
    return fail(ZKV_EINVAL, "zkv_h2d_gather: %s is not pinned, mapped host memory (%s)", name,
                hipGetErrorString(e));
  }
  if ((reinterpret_cast<uintptr_t>(d) & 15) != 0)
    return fail(ZKV_EINVAL, "zkv_h2d_gather: %s must be 16-byte aligned", name);
  *out = static_cast<const u32x4_t*>(d);
  return ZKV_OK;
}

}  // namespace
}  // namespace zkv

using namespace zkv;

extern "C" int zkv_h2d_gather_kv(const void* src_k, const void* src_v, int bs, int heads, int src_len,
                                 const int64_t* indices, int topk, void* dst_k, void* dst_v, int dst_len,
                                 zkv_stream_t stream) {
  ZKV_REQUIRE(src_k && src_v && indices && dst_k && dst_v, "zkv_h2d_gather_kv: null pointer");
  ZKV_REQUIRE(bs > 0 && heads > 0 && src_len > 0 && topk >= 0 && dst_len >= topk,
              "zkv_h2d_gather_kv: bad sizes bs=%d heads=%d src_len=%d topk=%d dst_len=%d", bs, heads,
              src_len, topk, dst_len);
  ZKV_REQUIRE((reinterpret_cast<uintptr_t>(dst_k) & 15) == 0 && (reinterpret_cast<uintptr_t>(dst_v) & 15) == 0,
              "zkv_h2d_gather_kv: destinations must be 16-byte aligned");
  if (topk == 0) return ZKV_OK;
  const u32x4_t *sk = nullptr, *sv = nullptr;
  if (int rc = device_alias(src_k, "src_k", &sk)) return rc;
  if (int rc = device_alias(src_v, "src_v", &sv)) return rc;
  const int64_t n_rows = static_cast<int64_t>(bs) * heads * topk;
  dim3 grid(static_cast<unsigned>((n_rows + 15) / 16), 1, 2);
  h2d_gather_kernel<<<grid, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      sk, sv, src_len, indices, topk, static_cast<u32x4_t*>(dst_k), static_cast<u32x4_t*>(dst_v), dst_len,
      n_rows);
  return check_launch("h2d_gather_kernel");
}

extern "C" int zkv_h2d_gather_kv_packed(const void* src_k, const void* src_v, int bs, int kv_heads,
                                        int src_len, void* dst_k_packed, void* dst_v_packed, int64_t total_k,
                                        const int64_t* indices_packed, int64_t total_topk,
                                        const int32_t* cu_seqlens_topk, const int32_t* cu_seqlens_k,
                                        int sl_end, int global_k, zkv_stream_t stream) {
  ZKV_REQUIRE(src_k && src_v && dst_k_packed && dst_v_packed && indices_packed && cu_seqlens_topk &&
                  cu_seqlens_k,
              "zkv_h2d_gather_kv_packed: null pointer");
  ZKV_REQUIRE(bs > 0 && kv_heads > 0 && src_len > 0 && total_k >= 0 && total_topk >= 0 && sl_end >= 0 &&
                  global_k >= 0,
              "zkv_h2d_gather_kv_packed: bad sizes");
  ZKV_REQUIRE((reinterpret_cast<uintptr_t>(dst_k_packed) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(dst_v_packed) & 15) == 0,
              "zkv_h2d_gather_kv_packed: destinations must be 16-byte aligned");
  if (global_k == 0) return ZKV_OK;
  const u32x4_t *sk = nullptr, *sv = nullptr;
  if (int rc = device_alias(src_k, "src_k", &sk)) return rc;
  if (int rc = device_alias(src_v, "src_v", &sv)) return rc;
  dim3 grid(static_cast<unsigned>(bs * kv_heads), static_cast<unsigned>((global_k + 15) / 16), 2);
  h2d_gather_packed_kernel<<<grid, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      sk, sv, kv_heads, src_len, static_cast<u32x4_t*>(dst_k_packed), static_cast<u32x4_t*>(dst_v_packed),
      total_k, indices_packed, total_topk, cu_seqlens_topk, cu_seqlens_k, sl_end);
  return check_launch("h2d_gather_packed_kernel");
}

// Pitched copy of `rows` rows of row_bytes each, any direction (device or
// pinned host on either side), on the stream's copy engine: the offload
// flush moves the oldest near-zone tokens of every (b, kv head) into their
// rows of the pinned host retrieval zone in one call.
extern "C" int zkv_copy_rows(void* dst, size_t dst_pitch, const void* src, size_t src_pitch, size_t row_bytes,
                             size_t rows, zkv_stream_t stream) {
  ZKV_REQUIRE(dst && src, "zkv_copy_rows: null pointer");
  ZKV_REQUIRE(row_bytes <= dst_pitch && row_bytes <= src_pitch,
              "zkv_copy_rows: row_bytes %zu exceeds a pitch (dst %zu, src %zu)", row_bytes, dst_pitch, src_pitch);
  if (rows == 0 || row_bytes == 0) return ZKV_OK;
  const hipError_t e = hipMemcpy2DAsync(dst, dst_pitch, src, src_pitch, row_bytes, rows, hipMemcpyDefault,
                                        reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(ZKV_ELAUNCH, "zkv_copy_rows: %s", hipGetErrorString(e));
  return ZKV_OK;
}

// Pinned (page-locked, device-mapped) host memory of exactly `bytes`: the
// offload retrieval zone.  (torch's pinned allocator rounds each block up to
// a power of two, which at C5 -- 72 blocks of 539 MB -- doubles the pinned
// footprint.)
extern "C" int zkv_host_alloc(size_t bytes, void** out) {
  ZKV_REQUIRE(out, "zkv_host_alloc: null output pointer");
  *out = nullptr;
  ZKV_REQUIRE(bytes > 0, "zkv_host_alloc: zero bytes");
  const hipError_t e = hipHostMalloc(out, bytes, hipHostMallocDefault);
  if (e != hipSuccess) {
    *out = nullptr;
    return fail(ZKV_ESPACE, "zkv_host_alloc: %zu bytes: %s", bytes, hipGetErrorString(e));
  }
  return ZKV_OK;
}

extern "C" int zkv_host_free(void* p) {
  if (p == nullptr) return ZKV_OK;
  const hipError_t e = hipHostFree(p);
  if (e != hipSuccess) return fail(ZKV_EINVAL, "zkv_host_free: %s", hipGetErrorString(e));
  return ZKV_OK;
}
