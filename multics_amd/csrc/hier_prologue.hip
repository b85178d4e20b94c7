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
// heads (the full model dim), so one workgroup owns whole tokens of one
// projection (q or k): dim/CPT threads x CPT channels (CPT = 4 up to dim 3072,
// else 8).  Camera weights stay in registers, packed, and the workgroup's
// camera rows in LDS, while the workgroup walks kTokens tokens two at a time:
// one workgroup reduction serves both tokens, each packed weight pair feeds
// both (v_dot2_f32_bf16), and the next two tokens' projections are loaded
// while the current two are computed.  The q workgroups also copy V into the
// requested layout.
#include "hier_common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
constexpr int kTokens = 32;

__device__ __forceinline__ float bf2f(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ uint32_t f2bf(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// Sums of NV values over the workgroup (blockDim a multiple of 64 or a power
// of two below 64); red holds 16 waves x NV partial sums.
template <int NV>
__device__ __forceinline__ void block_sum(float* v, float* red) {
  const int width = blockDim.x < 64 ? (int)blockDim.x : 64;
  for (int d = 1; d < width; d <<= 1)
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] += __shfl_xor(v[i], d, 64);
  const int nw = (blockDim.x + 63) >> 6;
  const int w = threadIdx.x >> 6;
  __syncthreads();   // the previous sums have been read
  if ((threadIdx.x & 63) == 0)
#pragma unroll
    for (int i = 0; i < NV; ++i) red[w * NV + i] = v[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    float t = 0.f;
    for (int ww = 0; ww < nw; ++ww) t += red[ww * NV + i];
    v[i] = t;
  }
}

// CPT channels per thread: 4 for model dims up to 3072, 8 up to 4096.
template <int CPT>
struct Chw;
template <>
struct Chw<4> { typedef u32x2 type; };
template <>
struct Chw<8> { typedef u32x4 type; };

// blockIdx.y selects the projection: 0 = q (and the V copy), 1 = k.  Keeping
// the two on separate workgroups halves the camera weights each thread holds,
// which lets two workgroups share a CU.
template <int C, int kCPT>
__global__ __launch_bounds__(kCPT == 4 ? 768 : 512) void prologue_kernel(HierPrologueArgs a) {
  typedef typename Chw<kCPT>::type chw_t;
  constexpr int CW = C > 0 ? C / 2 : 1;          // packed camera words per token
  __shared__ float red[16 * 2];
  __shared__ uint32_t camw[kTokens * CW];        // this workgroup's camera rows
  const bool is_k = blockIdx.y != 0;
  const uint16_t* const xin = is_k ? a.kx : a.qx;
  uint16_t* const out = is_k ? a.k_out : a.q_out;
  const bool copy_v = !is_k && a.v_out != nullptr;
  const int dim = a.H * a.D;
  const int c0 = threadIdx.x * kCPT;        // first channel of this thread
  const int head = c0 / a.D, d0 = c0 - head * a.D;
  const int half = a.D / 2;
  const int m0 = d0 / 2;
  const int s_begin = blockIdx.x * kTokens;
  const int s_end = min(a.S, s_begin + kTokens);

  // camera weights of this thread's kCPT channels: rows c0.. of [dim][C] are
  // contiguous, loaded as packed bf16 pairs (word i = elements 2i, 2i+1)
  constexpr int NW = C > 0 ? kCPT * C / 8 : 1;     // 16-byte vectors
  u32x4 wc[NW];
  if constexpr (C > 0) {
    const uint16_t* const w = is_k ? a.w_cam_k : a.w_cam_q;
#pragma unroll
    for (int i = 0; i < NW; ++i)
      wc[i] = *reinterpret_cast<const u32x4*>(w + (int64_t)c0 * C + 8 * i);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(a.cam + (int64_t)s_begin * C);
    for (int i = threadIdx.x; i < (s_end - s_begin) * CW; i += blockDim.x) camw[i] = src[i];
  }
  float g[kCPT];
  {
    const chw_t g4 = *reinterpret_cast<const chw_t*>((is_k ? a.norm_k_w : a.norm_q_w) + c0);
#pragma unroll
    for (int e = 0; e < kCPT / 2; ++e) {
      g[2 * e] = bf2f(g4[e] & 0xffffu);
      g[2 * e + 1] = bf2f(g4[e] >> 16);
    }
  }
  auto load = [&](int s) { return *reinterpret_cast<const chw_t*>(xin + (int64_t)s * dim + c0); };
  if constexpr (C > 0) __syncthreads();   // camera rows staged

  // Two tokens per trip (one reduction for both, each packed camera weight pair
  // feeds both), the next two tokens' projections loaded during the current
  // ones.  An odd last token is paired with itself and stored once.
  chw_t n0 = load(s_begin), n1 = load(min(s_begin + 1, s_end - 1));
  for (int s = s_begin; s < s_end; s += 2) {
    const chw_t x[2] = {n0, n1};
    const bool second = s + 1 < s_end;
    const int s1 = second ? s + 1 : s;
    typedef float rope_t __attribute__((ext_vector_type(kCPT / 2)));
    rope_t cs[2], sn[2];
    chw_t v4[2];
    cs[0] = *reinterpret_cast<const rope_t*>(a.rope_cos + (int64_t)s * half + m0);
    sn[0] = *reinterpret_cast<const rope_t*>(a.rope_sin + (int64_t)s * half + m0);
    cs[1] = *reinterpret_cast<const rope_t*>(a.rope_cos + (int64_t)s1 * half + m0);
    sn[1] = *reinterpret_cast<const rope_t*>(a.rope_sin + (int64_t)s1 * half + m0);
    if (copy_v) {
      v4[0] = *reinterpret_cast<const chw_t*>(a.vx + (int64_t)s * dim + c0);
      v4[1] = *reinterpret_cast<const chw_t*>(a.vx + (int64_t)s1 * dim + c0);
    }
    if (s + 2 < s_end) {
      n0 = load(s + 2);
      n1 = load(min(s + 3, s_end - 1));
    }
    float q[2][kCPT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < kCPT / 2; ++e) {
        q[t][2 * e] = bf2f(x[t][e] & 0xffffu);
        q[t][2 * e + 1] = bf2f(x[t][e] >> 16);
      }
    if constexpr (C > 0) {
      // packed bf16 pairs straight into v_dot2_f32_bf16: weight word w holds
      // elements (e, 2c), (e, 2c+1), camera word c holds cam[2c], cam[2c+1];
      // the products are exact in fp32 and accumulate in c order
      const uint32_t* cr[2] = {camw + (s - s_begin) * CW, camw + (s1 - s_begin) * CW};
#pragma unroll
      for (int e = 0; e < kCPT; ++e) {
        float acc[2] = {0.f, 0.f};
#pragma unroll
        for (int c = 0; c < CW; ++c) {
          const int w = e * CW + c;
          // (through a scalar temporary: a bit-cast applied to a vector
          // element subscript directly reads element 0)
          const uint32_t uw = wc[w >> 2][w & 3];
          const bf16x2 xw = __builtin_bit_cast(bf16x2, uw);
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const uint32_t uc = cr[t][c];
            acc[t] = __builtin_amdgcn_fdot2_f32_bf16(xw, __builtin_bit_cast(bf16x2, uc), acc[t],
                                                     false);
          }
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) q[t][e] = rbf(q[t][e] + rbf(acc[t]));
      }
    }
    float ss[2] = {0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < kCPT; ++e) ss[t] = fmaf(q[t][e], q[t][e], ss[t]);
    block_sum<2>(ss, red);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (t == 1 && !second) break;
      const float inv = rsqrtf(ss[t] / (float)dim + a.eps);
#pragma unroll
      for (int e = 0; e < kCPT; ++e) q[t][e] = rbf(rbf(q[t][e] * inv) * g[e]);
      // RoPE on (even, odd) channel pairs of this head
      chw_t qv;
#pragma unroll
      for (int e = 0; e < kCPT / 2; ++e) {
        const float c = cs[t][e], sv = sn[t][e];
        const float qr = q[t][2 * e] * c - q[t][2 * e + 1] * sv;
        const float qi = q[t][2 * e] * sv + q[t][2 * e + 1] * c;
        qv[e] = f2bf(qr) | (f2bf(qi) << 16);
      }
      const int64_t off = (int64_t)(s + t) * a.out_stride_s + (int64_t)head * a.out_stride_h + d0;
      *reinterpret_cast<chw_t*>(out + off) = qv;
      if (copy_v) *reinterpret_cast<chw_t*>(a.v_out + off) = v4[t];
    }
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
  const int kCPT = dim <= 3072 ? 4 : 8;
  const int nthr = dim / kCPT;
  HIER_REQUIRE(dim % kCPT == 0 && nthr <= (kCPT == 4 ? 768 : 512) && nthr >= 8 &&
                   (nthr % 64 == 0 || (nthr < 64 && (nthr & (nthr - 1)) == 0)),
               HIER_EUNSUPPORTED,
               "model dim %d must be a multiple of 256 up to 3072, of 512 up to 4096, or a power "
               "of two of at least 32",
               dim);
  HIER_REQUIRE(a.qx && a.kx && a.norm_q_w && a.norm_k_w && a.rope_cos && a.rope_sin && a.q_out &&
                   a.k_out && (!a.v_out || a.vx),
               HIER_EINVAL, "NULL tensor pointer");
  HIER_REQUIRE(a.out_stride_s % kCPT == 0 && a.out_stride_h % kCPT == 0, HIER_EINVAL,
               "output strides must keep %d-byte alignment", 2 * kCPT);
  const bool cam = a.cam != nullptr;
  HIER_REQUIRE(!cam || (a.C == 12 && a.w_cam_q && a.w_cam_k), HIER_EUNSUPPORTED,
               "camera adapter supports C=12 with both weights, got C=%d", a.C);
  HIER_REQUIRE(((uintptr_t)a.rope_cos & 15u) == 0 && ((uintptr_t)a.rope_sin & 15u) == 0 &&
                   (!cam || ((uintptr_t)a.cam & 7u) == 0),
               HIER_EINVAL, "RoPE tables must be 16-byte and camera rows 8-byte aligned");
  if (a.S == 0) return HIER_OK;
  const int grid = (a.S + kTokens - 1) / kTokens;
  const int threads = nthr;
  const hipStream_t st = (hipStream_t)stream;
  if (kCPT == 4) {
    if (cam) hipLaunchKernelGGL((prologue_kernel<12, 4>), dim3(grid, 2), dim3(threads), 0, st, a);
    else hipLaunchKernelGGL((prologue_kernel<0, 4>), dim3(grid, 2), dim3(threads), 0, st, a);
  } else {
    if (cam) hipLaunchKernelGGL((prologue_kernel<12, 8>), dim3(grid, 2), dim3(threads), 0, st, a);
    else hipLaunchKernelGGL((prologue_kernel<0, 8>), dim3(grid, 2), dim3(threads), 0, st, a);
  }
  return hier::check_launch("prologue_kernel");
}
