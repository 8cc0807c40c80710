// KV-cache writes: decode-step append and batched page fork copies.
//
// Layer layout [num_pages, 2, page_size, num_kv_heads, head_dim] (K at 0, V
// at 1), the reference's FlashInfer NHD paged layout (page_table.py:62-72).

#include <stdarg.h>

#include "common.h"

namespace be {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

// One thread moves 16 bytes (VEC = uint4) or one element (VEC = element type).
// Row = one (entry, head) of head_dim elements; rows_per = num_kv_heads.
template <typename VEC>
__global__ __launch_bounds__(256) void kv_append_kernel(char* kv, int num_pages, int page_size, int hkv,
                                                       int row_bytes, const int32_t* page_idx,
                                                       const int32_t* pos, const char* k, int64_t k_sn,
                                                       int64_t k_sh, const char* v, int64_t v_sn,
                                                       int64_t v_sh, int n, int32_t* err) {
  constexpr int VB = sizeof(VEC);
  const int per_row = row_bytes / VB;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)n * hkv * per_row;
  if (gid >= total) return;
  const int c = (int)(gid % per_row);
  const int h = (int)((gid / per_row) % hkv);
  const int i = (int)(gid / ((int64_t)per_row * hkv));
  const int p = page_idx[i], s = pos[i];
  if (p < 0 || p >= num_pages || s < 0 || s >= page_size) {
    if (err && c == 0 && h == 0) atomicAdd(err, 1);
    return;
  }
  const int64_t plane = (int64_t)page_size * hkv * row_bytes;          // bytes of K (or V) of one page
  const int64_t dst = (int64_t)p * 2 * plane + ((int64_t)s * hkv + h) * row_bytes + (int64_t)c * VB;
  const VEC kx = *reinterpret_cast<const VEC*>(k + i * k_sn + h * k_sh + (int64_t)c * VB);
  const VEC vx = *reinterpret_cast<const VEC*>(v + i * v_sn + h * v_sh + (int64_t)c * VB);
  *reinterpret_cast<VEC*>(kv + dst) = kx;
  *reinterpret_cast<VEC*>(kv + dst + plane) = vx;
}

// grid.x = copy entry c, grid.y = layer * 2 + kv.  Copies len[c] * hkv * row
// bytes (the first len slots are contiguous inside a page).  count (device,
// optional): entries c >= *count are skipped (a launch of fixed size whose
// live count is written on the device, e.g. inside a captured graph).
__global__ __launch_bounds__(256) void page_copy_kernel(char* pool, int64_t layer_stride, int num_pages,
                                                       int page_size, int64_t slot_bytes,
                                                       const int32_t* src, const int32_t* dst,
                                                       const int32_t* len, const int32_t* count, int vec,
                                                       int32_t* err) {
  const int c = blockIdx.x;
  if (count && c >= *count) return;
  const int layer = blockIdx.y >> 1, sel = blockIdx.y & 1;
  const int s = src[c], d = dst[c], l = len[c];
  if (s < 0 || s >= num_pages || d < 0 || d >= num_pages || l < 0 || l > page_size) {
    if (err && threadIdx.x == 0 && blockIdx.y == 0) atomicAdd(err, 1);
    return;
  }
  const int64_t plane = (int64_t)page_size * slot_bytes;
  const char* sp = pool + layer * layer_stride + ((int64_t)s * 2 + sel) * plane;
  char* dp = pool + layer * layer_stride + ((int64_t)d * 2 + sel) * plane;
  const int64_t bytes = (int64_t)l * slot_bytes;
  if (vec) {
    const int64_t nv = bytes >> 4;
    for (int64_t i = threadIdx.x; i < nv; i += 256)
      reinterpret_cast<uint4*>(dp)[i] = reinterpret_cast<const uint4*>(sp)[i];
  } else {
    for (int64_t i = threadIdx.x; i < bytes; i += 256) dp[i] = sp[i];
  }
}

}  // namespace be

extern "C" {

int be_version(void) { return 100; }   // 0.1.0

const char* be_last_error(void) { return be::g_last_error.c_str(); }

int be_kv_append(void* kv_layer, int dtype, int num_pages, int page_size, int num_kv_heads, int head_dim,
                 const int32_t* page_idx, const int32_t* pos, const void* k, int64_t k_stride_n,
                 int64_t k_stride_h, const void* v, int64_t v_stride_n, int64_t v_stride_h, int n,
                 int32_t* err_count, void* stream) {
  BE_REQUIRE(n >= 0, "n must be >= 0");
  if (n == 0) return BE_OK;
  BE_REQUIRE(kv_layer && page_idx && pos && k && v, "null pointer");
  BE_REQUIRE(dtype == BE_F32 || dtype == BE_F16 || dtype == BE_BF16, "unknown dtype %d", dtype);
  BE_REQUIRE(num_pages > 0 && page_size > 0 && num_kv_heads > 0 && head_dim > 0, "bad cache shape");
  const int64_t es = (int64_t)be::dtype_size(dtype);
  const int row_bytes = (int)(head_dim * es);
  const int64_t ksn = k_stride_n * es, ksh = k_stride_h * es, vsn = v_stride_n * es, vsh = v_stride_h * es;
  const bool vec = ((row_bytes & 15) == 0) && (((uintptr_t)kv_layer & 15) == 0) && (((uintptr_t)k & 15) == 0) &&
                   (((uintptr_t)v & 15) == 0) && ((ksn | ksh | vsn | vsh) & 15) == 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int vb = vec ? 16 : (int)es;
  const int64_t total = (int64_t)n * num_kv_heads * (row_bytes / vb);
  const unsigned blocks = (unsigned)((total + 255) / 256);
  char* kvp = reinterpret_cast<char*>(kv_layer);
  const char* kp = reinterpret_cast<const char*>(k);
  const char* vp = reinterpret_cast<const char*>(v);
  if (vec)
    be::kv_append_kernel<uint4><<<blocks, 256, 0, st>>>(kvp, num_pages, page_size, num_kv_heads, row_bytes, page_idx,
                                                       pos, kp, ksn, ksh, vp, vsn, vsh, n, err_count);
  else if (es == 4)
    be::kv_append_kernel<uint32_t><<<blocks, 256, 0, st>>>(kvp, num_pages, page_size, num_kv_heads, row_bytes,
                                                          page_idx, pos, kp, ksn, ksh, vp, vsn, vsh, n, err_count);
  else
    be::kv_append_kernel<uint16_t><<<blocks, 256, 0, st>>>(kvp, num_pages, page_size, num_kv_heads, row_bytes,
                                                          page_idx, pos, kp, ksn, ksh, vp, vsn, vsh, n, err_count);
  BE_HIP_CHECK(hipGetLastError());
  return BE_OK;
}

static int page_copy_launch(void* kv_pool, int64_t layer_stride_bytes, int num_layers, int dtype, int num_pages,
                            int page_size, int num_kv_heads, int head_dim, const int32_t* src, const int32_t* dst,
                            const int32_t* len, const int32_t* count, int n, int32_t* err_count, void* stream) {
  BE_REQUIRE(n >= 0 && num_layers >= 0, "negative count");
  if (n == 0 || num_layers == 0) return BE_OK;
  BE_REQUIRE(kv_pool && src && dst && len, "null pointer");
  BE_REQUIRE(dtype == BE_F32 || dtype == BE_F16 || dtype == BE_BF16, "unknown dtype %d", dtype);
  BE_REQUIRE(num_pages > 0 && page_size > 0 && num_kv_heads > 0 && head_dim > 0, "bad cache shape");
  const int64_t slot_bytes = (int64_t)num_kv_heads * head_dim * be::dtype_size(dtype);
  BE_REQUIRE(layer_stride_bytes >= (int64_t)num_pages * 2 * page_size * slot_bytes || num_layers == 1,
             "layer stride %lld smaller than one layer", (long long)layer_stride_bytes);
  BE_REQUIRE(num_layers <= 32767, "too many layers");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int vec = ((slot_bytes & 15) == 0) && ((layer_stride_bytes & 15) == 0) && (((uintptr_t)kv_pool & 15) == 0);
  be::page_copy_kernel<<<dim3(n, num_layers * 2), 256, 0, st>>>(reinterpret_cast<char*>(kv_pool), layer_stride_bytes,
                                                                num_pages, page_size, slot_bytes, src, dst, len, count,
                                                                vec, err_count);
  BE_HIP_CHECK(hipGetLastError());
  return BE_OK;
}

int be_page_copy(void* kv_pool, int64_t layer_stride_bytes, int num_layers, int dtype, int num_pages,
                 int page_size, int num_kv_heads, int head_dim, const int32_t* src, const int32_t* dst,
                 const int32_t* len, int n, int32_t* err_count, void* stream) {
  return page_copy_launch(kv_pool, layer_stride_bytes, num_layers, dtype, num_pages, page_size, num_kv_heads,
                          head_dim, src, dst, len, nullptr, n, err_count, stream);
}

int be_page_copy_counted(void* kv_pool, int64_t layer_stride_bytes, int num_layers, int dtype, int num_pages,
                         int page_size, int num_kv_heads, int head_dim, const int32_t* src, const int32_t* dst,
                         const int32_t* len, const int32_t* count, int max_n, int32_t* err_count, void* stream) {
  BE_REQUIRE(count, "null count");
  return page_copy_launch(kv_pool, layer_stride_bytes, num_layers, dtype, num_pages, page_size, num_kv_heads,
                          head_dim, src, dst, len, count, max_n, err_count, stream);
}

}  // extern "C"
