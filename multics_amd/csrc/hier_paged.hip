// Paged KV cache append: scatter the K/V rows of a cached block into their
// pool rows (one 16-byte chunk per thread, both tensors in one launch).
// HBM-bound copy; no row of the pool ever moves afterwards.
#include "hier_common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void kv_append_kernel(HierPageArgs a, int64_t total) {
  const int cpr = a.D / 8;                       // 16-byte chunks per (row, head)
  const int64_t per_row = (int64_t)a.H * cpr;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t row = i / per_row;
    const int64_t rem = i - row * per_row;
    const int h = (int)(rem / cpr), c = (int)(rem - (int64_t)h * cpr);
    const int dst = a.dst_rows[row];
    if (dst < 0 || dst >= a.pool_rows) continue;
    const int64_t po = (int64_t)dst * a.pool_ss + (int64_t)h * a.pool_sh + 8 * c;
    *reinterpret_cast<u32x4*>(a.k_pool + po) =
        *reinterpret_cast<const u32x4*>(a.k_src + row * a.k_src_ss + (int64_t)h * a.k_src_sh + 8 * c);
    *reinterpret_cast<u32x4*>(a.v_pool + po) =
        *reinterpret_cast<const u32x4*>(a.v_src + row * a.v_src_ss + (int64_t)h * a.v_src_sh + 8 * c);
  }
}

}  // namespace

extern "C" int hier_kv_append(const HierPageArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  const HierPageArgs& a = *args;
  HIER_REQUIRE(a.H >= 1 && a.D >= 8 && a.D % 8 == 0 && a.n_rows >= 0 && a.pool_rows >= 0,
               HIER_EINVAL, "invalid H=%d D=%d n_rows=%d pool_rows=%d", a.H, a.D, a.n_rows,
               a.pool_rows);
  if (a.n_rows == 0) return HIER_OK;
  HIER_REQUIRE(a.k_src && a.v_src && a.dst_rows && a.k_pool && a.v_pool, HIER_EINVAL,
               "NULL pointer");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  HIER_REQUIRE(al16(a.k_src) && al16(a.v_src) && al16(a.k_pool) && al16(a.v_pool), HIER_EINVAL,
               "K/V rows must be 16-byte aligned");
  HIER_REQUIRE(a.k_src_ss % 8 == 0 && a.k_src_sh % 8 == 0 && a.v_src_ss % 8 == 0 &&
                   a.v_src_sh % 8 == 0 && a.pool_ss % 8 == 0 && a.pool_sh % 8 == 0,
               HIER_EINVAL, "strides must keep 16-byte rows aligned");
  const int64_t total = (int64_t)a.n_rows * a.H * (a.D / 8);
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  const int grid = (int)(blocks < 65536 ? blocks : 65536);
  hipLaunchKernelGGL(kv_append_kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, a,
                     total);
  return hier::check_launch("kv_append_kernel");
}
