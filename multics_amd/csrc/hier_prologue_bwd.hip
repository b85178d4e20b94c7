// Backward of the Q/K projection tail (camera add, RMSNorm, gain, RoPE):
// the autograd of SelfAttention._project_self_attn_qkv after the three GEMMs
// (multics/models/attention.py:355-365, 307-320, 231-242; rope.py:248-254).
//
// Forward, per token and projection (x = q(x) or k(x), dim = H * D):
//   a = bf16(x + bf16(cam . Wc^T))      camera adapter (when present)
//   r = rsqrt(mean(a^2) + eps)
//   y = bf16(a * r),  z = bf16(y * w),  out = bf16(rotate(z, theta))
// Backward, given d_out:
//   dz = rotate(d_out, -theta)                    (the rotation's transpose)
//   dw += dz * y                                  (gain gradient, summed over tokens)
//   dy = dz * w
//   da = r * dy - r^3 * a * sum(dy * a) / dim     (RMSNorm)
//   dx = da                                       (the add passes it through)
// in fp32 from the saved inputs: a, r and y are recomputed from x, the camera
// row and the weights (the forward keeps nothing extra).  The camera-weight
// gradient dWc = dx^T . cam and the gain sums over waves are left to the
// caller (a plain GEMM and a column sum).
//
// One wave per run of `tpw` consecutive tokens of one projection
// (blockIdx.y: 0 = q, 1 = k); lane l holds the 8-channel chunks 8(64 j + l),
// j < NCH = dim / 512, which are 4 RoPE pairs of one head at the same pair
// index in every chunk (one cos and one sin float4 per token).  The two row
// sums (mean square, dy . a) are register sums plus a DPP wave reduction.  A
// token's camera row is shared by every token of its player's frame, so the
// camera product is recomputed only where the row changes.  Each wave writes
// its gain-gradient partial row (zeros for a wave without tokens).
#include "hier_common.h"

#include <algorithm>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float rbf(float x) {   // round to bf16 (nearest even) and back
  const f32x2 v = {0.f, x};
  return __uint_as_float(__builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2)));
}
__device__ __forceinline__ uint32_t pack(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Sum over the 64 lanes of a wave, in every lane (DPP rows of 16, then the
// 16- and 32-lane swaps of gfx950).
__device__ __forceinline__ float wsum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
  v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

template <int NCH, int C>
__global__ __launch_bounds__(256) void prologue_bwd_kernel(HierPrologueBwdArgs a, int tpw) {
  constexpr int dim = NCH * 512;
  constexpr int CW = C > 0 ? C / 2 : 1;
  const int lane = threadIdx.x & 63;
  const bool is_k = blockIdx.y != 0;
  const int wave_id = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int s_begin = wave_id * tpw;
  const int s_end = min(a.S, s_begin + tpw);
  const uint16_t* const xin = is_k ? a.kx : a.qx;
  const uint16_t* const dout = is_k ? a.dk : a.dq;
  const int64_t d_ss = is_k ? a.dk_ss : a.dq_ss, d_sh = is_k ? a.dk_sh : a.dq_sh;
  uint16_t* const dx = is_k ? a.dkx : a.dqx;
  const int D = a.D, half = D / 2;
  const int d0 = (8 * lane) % D;               // the same in every chunk (D divides 512)
  const int m0 = d0 / 2;
  const float inv_dim = 1.f / (float)dim;

  float g[NCH][8];                             // RMSNorm gains
  {
    const u32x4* gw = reinterpret_cast<const u32x4*>(is_k ? a.norm_k_w : a.norm_q_w) + lane;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const u32x4 w = gw[64 * j];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        g[j][2 * e] = lo(w[e]);
        g[j][2 * e + 1] = hi(w[e]);
      }
    }
  }
  float dw[NCH][8];
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) dw[j][e] = 0.f;
  uint32_t cp[NCH][4] = {};                    // camera product of the current row, packed bf16
  uint32_t camw_prev[CW] = {};

  for (int s = s_begin; s < s_end; ++s) {
    if constexpr (C > 0) {
      const uint32_t* cr = reinterpret_cast<const uint32_t*>(a.cam + (int64_t)s * C);
      uint32_t cw[CW];
      bool diff = s == s_begin;
#pragma unroll
      for (int c = 0; c < CW; ++c) {
        cw[c] = cr[c];
        diff = diff || cw[c] != camw_prev[c];
      }
      if (diff) {   // wave-uniform
#pragma unroll
        for (int c = 0; c < CW; ++c) camw_prev[c] = cw[c];
        const uint32_t* wbase = reinterpret_cast<const uint32_t*>(is_k ? a.w_cam_k : a.w_cam_q);
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
          float pr[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            // W[ch][2c], W[ch][2c + 1] packed in word c of row ch; exact
            // products, fp32 sums in c order (as the forward)
            const uint32_t* wr = wbase + (int64_t)(8 * (64 * j + lane) + e) * CW;
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < CW; ++c)
              acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wr[c]),
                                                    __builtin_bit_cast(bf16x2, cw[c]), acc, false);
            pr[e] = acc;
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) cp[j][e] = pack(pr[2 * e], pr[2 * e + 1]);
        }
      }
    }
    // a (camera added, bf16) and its mean square
    float av[NCH][8];
    float ss = 0.f;
    const u32x4* xr = reinterpret_cast<const u32x4*>(xin + (int64_t)s * dim + 8 * lane);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const u32x4 xv = xr[64 * j];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float x0 = lo(xv[e]), x1 = hi(xv[e]);
        if constexpr (C > 0) {
          x0 = rbf(x0 + lo(cp[j][e]));
          x1 = rbf(x1 + hi(cp[j][e]));
        }
        av[j][2 * e] = x0;
        av[j][2 * e + 1] = x1;
        ss = fmaf(x0, x0, fmaf(x1, x1, ss));
      }
    }
    const float r = __builtin_amdgcn_rsqf(wsum(ss) * inv_dim + a.eps);
    const float4 cs = *reinterpret_cast<const float4*>(a.rope_cos + (int64_t)s * half + m0);
    const float4 sn = *reinterpret_cast<const float4*>(a.rope_sin + (int64_t)s * half + m0);
    const float cv[4] = {cs.x, cs.y, cs.z, cs.w}, sv[4] = {sn.x, sn.y, sn.z, sn.w};
    // dz, the gain gradient, dy (kept in av's place as dyv) and sum(dy * a)
    float dyv[NCH][8];
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = 8 * (64 * j + lane);
      const u32x4 dv = *reinterpret_cast<const u32x4*>(dout + (int64_t)s * d_ss +
                                                        (int64_t)(c / D) * d_sh + d0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float q0 = lo(dv[e]), q1 = hi(dv[e]);
        const float z0 = q0 * cv[e] + q1 * sv[e];
        const float z1 = q1 * cv[e] - q0 * sv[e];
        const float y0 = rbf(av[j][2 * e] * r), y1 = rbf(av[j][2 * e + 1] * r);
        dw[j][2 * e] = fmaf(z0, y0, dw[j][2 * e]);
        dw[j][2 * e + 1] = fmaf(z1, y1, dw[j][2 * e + 1]);
        const float dy0 = z0 * g[j][2 * e], dy1 = z1 * g[j][2 * e + 1];
        dyv[j][2 * e] = dy0;
        dyv[j][2 * e + 1] = dy1;
        dot = fmaf(dy0, av[j][2 * e], fmaf(dy1, av[j][2 * e + 1], dot));
      }
    }
    const float kcoef = r * r * r * wsum(dot) * inv_dim;
    u32x4* xo = reinterpret_cast<u32x4*>(dx + (int64_t)s * dim + 8 * lane);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = pack(r * dyv[j][2 * e] - kcoef * av[j][2 * e],
                    r * dyv[j][2 * e + 1] - kcoef * av[j][2 * e + 1]);
      xo[64 * j] = o;
    }
  }
  // this wave's gain-gradient partial row
  float4* pr = reinterpret_cast<float4*>((is_k ? a.dw_k_partial : a.dw_q_partial) +
                                         (int64_t)wave_id * dim + 8 * lane);
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    pr[128 * j] = make_float4(dw[j][0], dw[j][1], dw[j][2], dw[j][3]);
    pr[128 * j + 1] = make_float4(dw[j][4], dw[j][5], dw[j][6], dw[j][7]);
  }
}

}  // namespace

extern "C" int hier_qk_prologue_bwd_waves(const HierPrologueBwdArgs* args) {
  if (!args || args->S < 0 || args->tokens_per_wave < 1) return -1;
  const int64_t waves = ((int64_t)args->S + args->tokens_per_wave - 1) / args->tokens_per_wave;
  return waves > (1ll << 28) ? -1 : (int)((waves + 3) / 4 * 4);   // whole workgroups of 4
}

extern "C" int hier_qk_prologue_bwd(const HierPrologueBwdArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  const HierPrologueBwdArgs& a = *args;
  HIER_REQUIRE(a.S >= 0 && a.H >= 1 && a.H <= 4096 && (a.D == 64 || a.D == 128) &&
                   a.tokens_per_wave >= 1,
               HIER_EUNSUPPORTED, "prologue backward supports head_dim 64/128, got H=%d D=%d",
               a.H, a.D);
  const int dim = a.H * a.D;
  const int nch = dim / 512;
  HIER_REQUIRE(dim % 512 == 0 && nch >= 1 && nch <= 8, HIER_EUNSUPPORTED,
               "prologue backward supports model dims that are multiples of 512 up to 4096, got %d",
               dim);
  HIER_REQUIRE(a.qx && a.kx && a.dq && a.dk && a.dqx && a.dkx && a.norm_q_w && a.norm_k_w &&
                   a.rope_cos && a.rope_sin && a.dw_q_partial && a.dw_k_partial,
               HIER_EINVAL, "NULL pointer");
  const bool cam = a.cam != nullptr;
  HIER_REQUIRE(!cam || (a.C == 12 && a.w_cam_q && a.w_cam_k), HIER_EUNSUPPORTED,
               "camera adapter supports C=12 with both weights, got C=%d", a.C);
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  HIER_REQUIRE(al16(a.qx) && al16(a.kx) && al16(a.dq) && al16(a.dk) && al16(a.dqx) &&
                   al16(a.dkx) && al16(a.norm_q_w) && al16(a.norm_k_w) && al16(a.rope_cos) &&
                   al16(a.rope_sin) && al16(a.dw_q_partial) && al16(a.dw_k_partial) &&
                   (!cam || (((uintptr_t)a.cam & 3u) == 0 && ((uintptr_t)a.w_cam_q & 3u) == 0 &&
                             ((uintptr_t)a.w_cam_k & 3u) == 0)),
               HIER_EINVAL, "tensors must be 16-byte aligned (camera rows and weights 4-byte)");
  HIER_REQUIRE(a.dq_ss >= 0 && a.dq_sh >= 0 && a.dk_ss >= 0 && a.dk_sh >= 0 && a.dq_ss % 8 == 0 &&
                   a.dq_sh % 8 == 0 && a.dk_ss % 8 == 0 && a.dk_sh % 8 == 0,
               HIER_EINVAL, "gradient strides must be non-negative multiples of 8");
  HIER_REQUIRE((int64_t)a.S * dim <= ((int64_t)1 << 40), HIER_EUNSUPPORTED, "too many tokens");
  if (a.S == 0) return HIER_OK;
  const int waves = hier_qk_prologue_bwd_waves(&a);
  HIER_REQUIRE(waves > 0, HIER_EUNSUPPORTED, "too many waves");
  const dim3 grid((waves + 3) / 4, 2);
  hipStream_t st = (hipStream_t)stream;
#define HIER_PBWD(N)                                                                          \
  if (nch == N) {                                                                             \
    if (cam) hipLaunchKernelGGL((prologue_bwd_kernel<N, 12>), grid, dim3(256), 0, st, a,       \
                                a.tokens_per_wave);                                           \
    else hipLaunchKernelGGL((prologue_bwd_kernel<N, 0>), grid, dim3(256), 0, st, a,           \
                            a.tokens_per_wave);                                               \
  }
  HIER_PBWD(1) HIER_PBWD(2) HIER_PBWD(3) HIER_PBWD(4) HIER_PBWD(5) HIER_PBWD(6) HIER_PBWD(7)
  HIER_PBWD(8)
#undef HIER_PBWD
  return hier::check_launch("prologue_bwd_kernel");
}
