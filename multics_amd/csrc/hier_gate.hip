// Gated residual of the DiT block after self-attention:
//   out = x + gate * y        (GateModule.forward, multics/models/blocks.py:31-35,
//                              applied at blocks.py:661, 668 to the o-projection
//                              output y with the per-(player, frame) gate_msa)
// The gate holds one row per `rows_per_gate` consecutive rows of x / y (a
// frame's L tokens share their player-frame's gate row, blocks.py:604-616),
// so it is read from a small table instead of being materialised at the
// size of x.  bf16 in and out; each element is computed as torch's bf16
// expression does -- the product rounded to bf16, then the sum rounded to
// bf16 -- so the result is bit-identical to it.
//
// One pass over HBM: x and y read once, out written once (out may be x).
// Each thread moves 16-byte chunks (8 channels); the grid strides over the
// rows x (dim / 8) chunks.
#include "hier_common.h"

#include <algorithm>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t rnd(float f) {   // round to nearest even, as torch
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ uint32_t gate_pair(uint32_t xw, uint32_t gw, uint32_t yw) {
  const float p0 = __uint_as_float(rnd(lo(gw) * lo(yw)) << 16);
  const float p1 = __uint_as_float(rnd(hi(gw) * hi(yw)) << 16);
  return rnd(lo(xw) + p0) | (rnd(hi(xw) + p1) << 16);
}

__global__ __launch_bounds__(256) void gate_kernel(HierGateArgs a, int64_t n_chunks, int cpr) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_chunks; i += stride) {
    const int64_t row = i / cpr;
    const int c = (int)(i - row * cpr);
    const int64_t grow = row / a.rows_per_gate;
    const u32x4 xv = *reinterpret_cast<const u32x4*>(a.x + row * a.x_ss + 8 * c);
    const u32x4 yv = *reinterpret_cast<const u32x4*>(a.y + row * a.y_ss + 8 * c);
    const u32x4 gv = *reinterpret_cast<const u32x4*>(a.gate + grow * a.gate_ss + 8 * c);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = gate_pair(xv[e], gv[e], yv[e]);
    *reinterpret_cast<u32x4*>(a.out + row * a.out_ss + 8 * c) = o;
  }
}

}  // namespace

extern "C" int hier_gated_residual(const HierGateArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  const HierGateArgs& a = *args;
  HIER_REQUIRE(a.rows >= 0 && a.dim >= 8 && a.dim % 8 == 0 && a.rows_per_gate >= 1, HIER_EINVAL,
               "invalid rows=%lld dim=%d rows_per_gate=%d", (long long)a.rows, a.dim,
               a.rows_per_gate);
  HIER_REQUIRE(a.x_ss >= a.dim && a.y_ss >= a.dim && a.gate_ss >= a.dim && a.out_ss >= a.dim &&
                   a.x_ss % 8 == 0 && a.y_ss % 8 == 0 && a.gate_ss % 8 == 0 && a.out_ss % 8 == 0,
               HIER_EINVAL, "row strides must be multiples of 8 of at least dim");
  if (a.rows == 0) return HIER_OK;
  HIER_REQUIRE(a.x && a.y && a.gate && a.out, HIER_EINVAL, "NULL pointer");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  HIER_REQUIRE(al16(a.x) && al16(a.y) && al16(a.gate) && al16(a.out), HIER_EINVAL,
               "x / y / gate / out must be 16-byte aligned");
  HIER_REQUIRE(a.rows <= (1ll << 40) / a.dim, HIER_EUNSUPPORTED, "too many elements");
  const int cpr = a.dim / 8;
  const int64_t n = a.rows * cpr;
  // about eight chunks per thread: enough loads in flight, few waves
  const int64_t blocks = std::min<int64_t>((n + 2047) / 2048, 256 * 32);
  hipLaunchKernelGGL(gate_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, a,
                     n, cpr);
  return hier::check_launch("gate_kernel");
}
