// Paged KV cache append: scatter the K/V rows of a cached block into their
// pool rows (16-byte chunks, both tensors in one launch).
// HBM-bound copy; no row of the pool ever moves afterwards.
#include "hier_common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

// One workgroup per block row: the destination row is read once, and each
// thread's (head, chunk) comes from 32-bit index arithmetic.
__global__ __launch_bounds__(kThreads) void kv_append_kernel(HierPageArgs a) {
  const int row = blockIdx.x;
  const int dst = a.dst_rows[row];
  if (dst < 0 || dst >= a.pool_rows) return;
  const int cpr = a.D / 8;                       // 16-byte chunks per (row, head)
  const int per_row = a.H * cpr;
  const uint16_t* ks = a.k_src + (int64_t)row * a.k_src_ss;
  const uint16_t* vs = a.v_src + (int64_t)row * a.v_src_ss;
  uint16_t* kd = a.k_pool + (int64_t)dst * a.pool_ss;
  uint16_t* vd = a.v_pool + (int64_t)dst * a.pool_ss;
  for (int j = threadIdx.x; j < per_row; j += kThreads) {
    const int h = j / cpr, c = j - h * cpr;
    const u32x4 kx = *reinterpret_cast<const u32x4*>(ks + (int64_t)h * a.k_src_sh + 8 * c);
    const u32x4 vx = *reinterpret_cast<const u32x4*>(vs + (int64_t)h * a.v_src_sh + 8 * c);
    const int64_t po = (int64_t)h * a.pool_sh + 8 * c;
    *reinterpret_cast<u32x4*>(kd + po) = kx;
    *reinterpret_cast<u32x4*>(vd + po) = vx;
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
  HIER_REQUIRE((int64_t)a.H * (a.D / 8) < (1ll << 31), HIER_EUNSUPPORTED, "rows too wide");
  hipLaunchKernelGGL(kv_append_kernel, dim3(a.n_rows), dim3(kThreads), 0, (hipStream_t)stream, a);
  return hier::check_launch("kv_append_kernel");
}
