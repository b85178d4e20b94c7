// Q/K/V layout prologue: camera-pose Q/K adapter + RMSNorm + gain + RoPE.
//
// Restates, fused into one HBM pass per token, the part of
// SelfAttention._project_self_attn_qkv that follows the three projection GEMMs
// (multics/models/attention.py:355-365):
//
//   qx += bf16(cam_q(cam))                      attention.py:307-320 (bias-free,
//   kx += bf16(cam_k(cam))                      compatible_linear.py:12-35)
//   q = bf16(bf16(qx * rsqrt(mean(qx^2) + eps)) * w_q)   RMSNorm, attention.py:231-242
//   q = bf16(rotate(q, freqs))                  rope_apply, rope.py:248-254
//
// with the same bf16 rounding points as the reference.  The reference rotates
// in float64; here the rotation runs in fp32 from fp32 cos/sin tables, so a
// result can differ from the reference by one bf16 ulp.  The RMS spans all
// heads (the full model dim), so one workgroup owns whole tokens: dim/8
// threads x 8 channels.  Camera weights stay in registers while the
// workgroup walks kTokens tokens.  V is copied into the requested layout.
#include "hier_common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kTokens = 32;

__device__ __forceinline__ float bf2f(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ uint32_t f2bf(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// Sum over the workgroup; blockDim is a multiple of 64 or a power of two below 64.
__device__ __forceinline__ float2 block_sum2(float2 v, float2* red) {
  const int width = blockDim.x < 64 ? (int)blockDim.x : 64;
  for (int d = 1; d < width; d <<= 1) {
    v.x += __shfl_xor(v.x, d, 64);
    v.y += __shfl_xor(v.y, d, 64);
  }
  const int nw = (blockDim.x + 63) >> 6;
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float2 t = make_float2(0.f, 0.f);
  for (int i = 0; i < nw; ++i) { t.x += red[i].x; t.y += red[i].y; }
  return t;
}

template <int C>
__global__ __launch_bounds__(512) void prologue_kernel(HierPrologueArgs a) {
  __shared__ float2 red[16];
  const int dim = a.H * a.D;
  const int c0 = threadIdx.x * 8;           // first channel of this thread
  const int head = c0 / a.D, d0 = c0 - head * a.D;
  const int half = a.D / 2;

  // camera weights of this thread's 8 channels: rows c0..c0+7 of [dim][C] are
  // contiguous, loaded as packed bf16 pairs (word i = elements 2i, 2i+1)
  constexpr int NW = C > 0 ? 8 * C / 8 : 1;     // 16-byte vectors
  u32x4 wq[NW], wk[NW];
  if constexpr (C > 0) {
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      wq[i] = *reinterpret_cast<const u32x4*>(a.w_cam_q + (int64_t)c0 * C + 8 * i);
      wk[i] = *reinterpret_cast<const u32x4*>(a.w_cam_k + (int64_t)c0 * C + 8 * i);
    }
  }
  float gq[8], gk[8];
  {
    const u32x4 q4 = *reinterpret_cast<const u32x4*>(a.norm_q_w + c0);
    const u32x4 k4 = *reinterpret_cast<const u32x4*>(a.norm_k_w + c0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      gq[2 * e] = bf2f(q4[e] & 0xffffu); gq[2 * e + 1] = bf2f(q4[e] >> 16);
      gk[2 * e] = bf2f(k4[e] & 0xffffu); gk[2 * e + 1] = bf2f(k4[e] >> 16);
    }
  }

  const int s_end = min(a.S, (int)(blockIdx.x + 1) * kTokens);
  for (int s = blockIdx.x * kTokens; s < s_end; ++s) {
    float q[8], k[8];
    {
      const u32x4 q4 = *reinterpret_cast<const u32x4*>(a.qx + (int64_t)s * dim + c0);
      const u32x4 k4 = *reinterpret_cast<const u32x4*>(a.kx + (int64_t)s * dim + c0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        q[2 * e] = bf2f(q4[e] & 0xffffu); q[2 * e + 1] = bf2f(q4[e] >> 16);
        k[2 * e] = bf2f(k4[e] & 0xffffu); k[2 * e + 1] = bf2f(k4[e] >> 16);
      }
    }
    if constexpr (C > 0) {
      // keep the weights packed: stops the unpack being hoisted out of the
      // token loop (it would need 2*8*C fp32 registers)
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        asm volatile("" : "+v"(wq[i]));
        asm volatile("" : "+v"(wk[i]));
      }
      float cam[C];
#pragma unroll
      for (int c = 0; c < C; ++c) cam[c] = bf2f(a.cam[(int64_t)s * C + c]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float aq = 0.f, ak = 0.f;
#pragma unroll
        for (int c = 0; c < C / 2; ++c) {
          const int w = (e * C) / 2 + c;     // packed word of elements (e, 2c), (e, 2c+1)
          const uint32_t xq = wq[w >> 2][w & 3], xk = wk[w >> 2][w & 3];
          aq = fmaf(cam[2 * c], __uint_as_float(xq << 16), aq);
          aq = fmaf(cam[2 * c + 1], __uint_as_float(xq & 0xffff0000u), aq);
          ak = fmaf(cam[2 * c], __uint_as_float(xk << 16), ak);
          ak = fmaf(cam[2 * c + 1], __uint_as_float(xk & 0xffff0000u), ak);
        }
        q[e] = rbf(q[e] + rbf(aq));
        k[e] = rbf(k[e] + rbf(ak));
      }
    }
    float2 ss = make_float2(0.f, 0.f);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ss.x = fmaf(q[e], q[e], ss.x);
      ss.y = fmaf(k[e], k[e], ss.y);
    }
    ss = block_sum2(ss, red);
    const float iq = rsqrtf(ss.x / (float)dim + a.eps);
    const float ik = rsqrtf(ss.y / (float)dim + a.eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      q[e] = rbf(rbf(q[e] * iq) * gq[e]);
      k[e] = rbf(rbf(k[e] * ik) * gk[e]);
    }
    // RoPE on (even, odd) channel pairs of this head
    uint32_t qo[4], ko[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = d0 / 2 + e;
      const float cs = a.rope_cos[(int64_t)s * half + m];
      const float sn = a.rope_sin[(int64_t)s * half + m];
      const float qr = q[2 * e] * cs - q[2 * e + 1] * sn;
      const float qi = q[2 * e] * sn + q[2 * e + 1] * cs;
      const float kr = k[2 * e] * cs - k[2 * e + 1] * sn;
      const float ki = k[2 * e] * sn + k[2 * e + 1] * cs;
      qo[e] = f2bf(qr) | (f2bf(qi) << 16);
      ko[e] = f2bf(kr) | (f2bf(ki) << 16);
    }
    const int64_t off = (int64_t)s * a.out_stride_s + (int64_t)head * a.out_stride_h + d0;
    u32x4 qv = {qo[0], qo[1], qo[2], qo[3]};
    u32x4 kv = {ko[0], ko[1], ko[2], ko[3]};
    *reinterpret_cast<u32x4*>(a.q_out + off) = qv;
    *reinterpret_cast<u32x4*>(a.k_out + off) = kv;
    if (a.v_out)
      *reinterpret_cast<u32x4*>(a.v_out + off) =
          *reinterpret_cast<const u32x4*>(a.vx + (int64_t)s * dim + c0);
  }
}

}  // namespace

extern "C" int hier_qkv_prologue(const HierPrologueArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  const HierPrologueArgs& a = *args;
  HIER_REQUIRE(a.S >= 0 && a.H >= 1 && (a.D == 64 || a.D == 128), HIER_EUNSUPPORTED,
               "prologue supports head_dim 64/128, got H=%d D=%d", a.H, a.D);
  const int dim = a.H * a.D;
  const int nthr = dim / 8;
  HIER_REQUIRE(dim % 8 == 0 && nthr <= 512 && nthr >= 8 &&
                   (nthr % 64 == 0 || (nthr < 64 && (nthr & (nthr - 1)) == 0)),
               HIER_EUNSUPPORTED, "model dim %d must be 8 x (a multiple of 64 up to 512, or a power of two)",
               dim);
  HIER_REQUIRE(a.qx && a.kx && a.norm_q_w && a.norm_k_w && a.rope_cos && a.rope_sin && a.q_out &&
                   a.k_out && (!a.v_out || a.vx),
               HIER_EINVAL, "NULL tensor pointer");
  HIER_REQUIRE(a.out_stride_s % 8 == 0 && a.out_stride_h % 8 == 0, HIER_EINVAL,
               "output strides must keep 16-byte alignment");
  const bool cam = a.cam != nullptr;
  HIER_REQUIRE(!cam || (a.C == 12 && a.w_cam_q && a.w_cam_k), HIER_EUNSUPPORTED,
               "camera adapter supports C=12 with both weights, got C=%d", a.C);
  if (a.S == 0) return HIER_OK;
  const int grid = (a.S + kTokens - 1) / kTokens;
  const int threads = dim / 8;
  if (cam)
    hipLaunchKernelGGL(prologue_kernel<12>, dim3(grid), dim3(threads), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(prologue_kernel<0>, dim3(grid), dim3(threads), 0, (hipStream_t)stream, a);
  return hier::check_launch("prologue_kernel");
}
