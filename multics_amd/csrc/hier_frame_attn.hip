// Frame-window attention of the action branches' cached attention
// (multics/models/blocks.py:256-375: mouse temporal self-attention and
// keyboard cross-attention over a rolling cache).  The sequences are short
// (a few queries per sequence and head against at most a few hundred cached
// keys), so instead of the tile kernel's 32 x 32 MFMA blocks a wave serves
// 64 / (D/8) (sequence, query) slots of one head: each query owns D/8 lanes,
// each lane 8 channels.  The partial dot products are summed across the
// query's lanes and the softmax runs online in fp32.  For the temporal
// branch the kernel is bound by reading the cached window once.
#include "hier_common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t f2bf(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

template <int D>
__global__ __launch_bounds__(64) void frame_attn_kernel(HierFrameAttnArgs a) {
  constexpr int LPQ = D / 8;          // lanes per query
  constexpr int QPW = 64 / LPQ;       // queries per wave
  // the wave's query slots run over (batch, query) pairs, so sequences with
  // fewer queries than slots share a wave; each slot reads its own
  // sequence's keys (slots of one sequence read the same rows)
  const int lane = threadIdx.x;
  const int c = lane % LPQ;
  const int slot = blockIdx.x * QPW + lane / LPQ;
  const int h = blockIdx.y;
  const bool valid = slot < a.B * a.Lq;
  const int b = valid ? slot / a.Lq : 0;
  const int qi = valid ? slot - b * a.Lq : 0;
  const int qs = qi;
  const u32x4 qw = *reinterpret_cast<const u32x4*>(a.q + b * a.q_sb + qs * a.q_ss + h * a.q_sh + 8 * c);
  const int qf = a.q_frame[qs];
  const int qblk = qf / a.n_block;
  const float c2 = a.scale * kLog2e;
  const uint16_t* kb = a.k + b * a.k_sb + h * a.k_sh + 8 * c;
  const uint16_t* vb = a.v + b * a.v_sb + h * a.v_sh + 8 * c;
  float m = -INFINITY, l = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // keys in groups of four: the group's rows are loaded before any is used,
  // so each wave keeps eight 16-byte loads in flight (groups of eight
  // measured slower)
  constexpr int G = 4;
  for (int j0 = 0; j0 < a.Lk; j0 += G) {
    u32x4 kwg[G], vwg[G];
    int kfg[G];
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const int j = min(j0 + u, a.Lk - 1);
      kwg[u] = *reinterpret_cast<const u32x4*>(kb + j * a.k_ss);
      vwg[u] = *reinterpret_cast<const u32x4*>(vb + j * a.v_ss);
      kfg[u] = a.k_frame[j];
    }
#pragma unroll
    for (int u = 0; u < G; ++u) {
      if (j0 + u >= a.Lk) break;
      const u32x4 kw = kwg[u], vw = vwg[u];
      const int kf = kfg[u];
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t x = qw[e], y = kw[e];
        s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x),
                                            __builtin_bit_cast(bf16x2, y), s, false);
      }
#pragma unroll
      for (int d = 1; d < LPQ; d <<= 1) s += __shfl_xor(s, d, 64);
      const bool vis =
          valid && kf / a.n_block <= qblk && (a.local_attn < 0 || qf - kf < a.local_attn);
      if (vis) {
        const float t = s * c2;
        const float mn = fmaxf(m, t);
        const float alpha = __builtin_amdgcn_exp2f(m - mn);   // m = -inf: 0
        const float p = __builtin_amdgcn_exp2f(t - mn);
        l = l * alpha + p;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t w = vw[e];
          o[2 * e] = fmaf(p, lo(w), o[2 * e] * alpha);
          o[2 * e + 1] = fmaf(p, hi(w), o[2 * e + 1] * alpha);
        }
        m = mn;
      }
    }
  }
  if (!valid) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  u32x4 ow;
#pragma unroll
  for (int e = 0; e < 4; ++e) ow[e] = f2bf(o[2 * e] * inv) | (f2bf(o[2 * e + 1] * inv) << 16);
  *reinterpret_cast<u32x4*>(a.o + b * a.o_sb + qi * a.o_ss + h * a.o_sh + 8 * c) = ow;
}

}  // namespace

extern "C" int hier_frame_attn(const HierFrameAttnArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  const HierFrameAttnArgs& a = *args;
  HIER_REQUIRE(a.D == 128 || a.D == 64, HIER_EUNSUPPORTED, "head_dim must be 64 or 128, got %d", a.D);
  HIER_REQUIRE(a.B >= 0 && a.Lq >= 0 && a.Lk >= 0 && a.H >= 1 && a.n_block >= 1 &&
                   a.local_attn >= -1 && a.local_attn != 0,
               HIER_EINVAL, "invalid B=%d Lq=%d Lk=%d H=%d n_block=%d local_attn=%d", a.B, a.Lq,
               a.Lk, a.H, a.n_block, a.local_attn);
  if (a.B == 0 || a.Lq == 0) return HIER_OK;
  HIER_REQUIRE(a.q && a.k && a.v && a.o && a.q_frame && (a.k_frame || a.Lk == 0), HIER_EINVAL,
               "NULL pointer");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  HIER_REQUIRE(al16(a.q) && al16(a.k) && al16(a.v) && al16(a.o), HIER_EINVAL,
               "q/k/v/o must be 16-byte aligned");
  HIER_REQUIRE(a.q_sb % 8 == 0 && a.q_ss % 8 == 0 && a.q_sh % 8 == 0 && a.k_sb % 8 == 0 &&
                   a.k_ss % 8 == 0 && a.k_sh % 8 == 0 && a.v_sb % 8 == 0 && a.v_ss % 8 == 0 &&
                   a.v_sh % 8 == 0 && a.o_sb % 8 == 0 && a.o_ss % 8 == 0 && a.o_sh % 8 == 0,
               HIER_EINVAL, "strides must keep 16-byte rows aligned");
  HIER_REQUIRE(a.H <= 65535, HIER_EUNSUPPORTED, "at most 65535 heads");
  const int qpw = 64 / (a.D / 8);
  const int64_t slots = (int64_t)a.B * a.Lq;
  HIER_REQUIRE(slots / qpw < (1ll << 31) - 1, HIER_EUNSUPPORTED, "too many queries");
  const dim3 grid((unsigned)((slots + qpw - 1) / qpw), a.H, 1);
  if (a.D == 128)
    hipLaunchKernelGGL(frame_attn_kernel<128>, grid, dim3(64), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(frame_attn_kernel<64>, grid, dim3(64), 0, (hipStream_t)stream, a);
  return hier::check_launch("frame_attn_kernel");
}
