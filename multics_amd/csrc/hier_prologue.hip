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
// heads (the full model dim), so each token of a projection (q or k) is owned
// whole by one wave or one workgroup:
//   * model dims that are multiples of 512 (up to 4096): row_prologue_kernel,
//     one wave per run of consecutive tokens, 8*NCH channels per lane, the RMS
//     a register sum plus one DPP wave reduction (no LDS traffic, no barrier
//     per token);
//   * other dims: prologue_kernel, one workgroup of dim/CPT threads x CPT
//     channels (CPT = 4 up to dim 3072, else 8) walking kTokens tokens two at
//     a time, one workgroup reduction (DPP and lane swaps inside each wave,
//     one LDS barrier across waves) per two tokens.
// Both load the next token's projection and RoPE rows into a second register
// set while the current one is computed.  A token's camera row is the same
// for every token of a player's frame (zero for hub tokens), so the camera
// product (v_dot2_f32_bf16 over packed bf16 pairs, weights read when needed)
// is recomputed only where the row changes.  With v_out the q waves /
// workgroups also copy V into the requested layout.
#include "hier_common.h"

#include <algorithm>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
constexpr int kTokens = 32;
constexpr int kTrip = 2;     // tokens per trip of the token loop

__device__ __forceinline__ float bf2f(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ uint32_t f2bf(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }
typedef float f32x2 __attribute__((ext_vector_type(2)));
// Both values rounded to bf16 (round to nearest even) and back: one
// v_cvt_pk_bf16_f32 for the pair, then a shift and a mask.
__device__ __forceinline__ void rbf2(float& a, float& b) {
  const f32x2 v = {a, b};
  const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  a = __uint_as_float(u << 16);
  b = __uint_as_float(u & 0xffff0000u);
}

// One value rounded to bf16 and back in one instruction: converting the pair
// (0, x) puts bf16(x) in the high half over a zero low half, which is the
// rounded value as an fp32.
__device__ __forceinline__ float rbf1(float x) {
  const f32x2 v = {0.f, x};
  return __uint_as_float(__builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2)));
}
// A pair of floats as packed bf16 (round to nearest even), one conversion.
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Sum over the 64 lanes of a wave, left in every lane: DPP within rows of
// 16, then the row swaps of gfx950 (v_permlane16_swap, v_permlane32_swap).
__device__ __forceinline__ float dpp_add(float v, int ctrl_sel) {
  int u;
  switch (ctrl_sel) {
    case 0: u = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false); break;
    case 1: u = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false); break;
    case 2: u = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false); break;
    default: u = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false); break;
  }
  return v + __int_as_float(u);
}
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add(v, 0);   // quad_perm [1,0,3,2]
  v = dpp_add(v, 1);   // quad_perm [2,3,0,1]
  v = dpp_add(v, 2);   // row_ror:4
  v = dpp_add(v, 3);   // row_ror:8
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
  v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// Sums of NV values over the workgroup.  Full waves (blockDim a multiple of
// 64): a register reduction per wave, then the wave sums through red, laid
// out [parity][NV][16 waves] with the slots of absent waves zero (the caller
// clears red once), so every value reads 16 slots unconditionally.  The two
// parity buffers alternate between calls, so one barrier per call suffices:
// the buffer a call writes was last read before the previous call's barrier.
// Below 64 threads (one partial wave): a shuffle reduction.
template <int NV>
__device__ __forceinline__ void block_sum(float* v, float* red, int parity) {
  if (blockDim.x >= 64) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = wave_sum(v[i]);
    float* r = red + parity * 16 * NV;
    if ((threadIdx.x & 63) == 0)
#pragma unroll
      for (int i = 0; i < NV; ++i) r[i * 16 + (threadIdx.x >> 6)] = v[i];
    hier::barrier_lds();   // (not __syncthreads: the next trip's prefetch stays in flight)
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const float4* r4 = reinterpret_cast<const float4*>(r + i * 16);
      float t = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 w = r4[j];
        t += (w.x + w.y) + (w.z + w.w);
      }
      v[i] = t;
    }
    return;
  }
  for (int d = 1; d < (int)blockDim.x; d <<= 1)
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] += __shfl_xor(v[i], d, 64);
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
template <int C, int kCPT, bool kCopyV>
__global__ __launch_bounds__(kCPT == 4 ? 768 : 512) void prologue_kernel(HierPrologueArgs a) {
  typedef typename Chw<kCPT>::type chw_t;
  typedef float rope_t __attribute__((ext_vector_type(kCPT / 2)));
  constexpr int CW = C > 0 ? C / 2 : 1;          // packed camera words per token
  __shared__ __align__(16) float red[2 * 16 * kTrip];
  __shared__ uint32_t camw[kTokens * CW];        // this workgroup's camera rows
  __shared__ uint8_t cam_new[kTokens];           // row differs from the previous token's
  const bool is_k = blockIdx.y != 0;
  const uint16_t* const xin = is_k ? a.kx : a.qx;
  uint16_t* const out = is_k ? a.k_out : a.q_out;
  const bool copy_v = kCopyV && !is_k;
  const int dim = a.H * a.D;
  const int c0 = threadIdx.x * kCPT;        // first channel of this thread
  const int head = c0 / a.D, d0 = c0 - head * a.D;
  const int half = a.D / 2;
  const int m0 = d0 / 2;
  const int s_begin = blockIdx.x * kTokens;
  const int s_end = min(a.S, s_begin + kTokens);
  const float inv_dim = 1.f / (float)dim;
  for (int i = threadIdx.x; i < 2 * 16 * kTrip; i += blockDim.x) red[i] = 0.f;
  if constexpr (C > 0) {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(a.cam + (int64_t)s_begin * C);
    for (int i = threadIdx.x; i < (s_end - s_begin) * CW; i += blockDim.x) camw[i] = src[i];
  }
  float g[kCPT];
  {
    const chw_t g4 = *reinterpret_cast<const chw_t*>((is_k ? a.norm_k_w : a.norm_q_w) + c0);
#pragma unroll
    for (int e = 0; e < kCPT / 2; ++e) {
      g[2 * e] = __uint_as_float(g4[e] << 16);
      g[2 * e + 1] = __uint_as_float(g4[e] & 0xffff0000u);
    }
  }
  // element offsets of the [S, dim] projections fit in 32 bits (checked by the launcher)
  auto load = [&](int s) {
    return *reinterpret_cast<const chw_t*>(xin + (uint32_t)(s * dim + c0));
  };
  auto rc = [&](int s) {
    return *reinterpret_cast<const rope_t*>(a.rope_cos + (uint32_t)(s * half + m0));
  };
  auto rs = [&](int s) {
    return *reinterpret_cast<const rope_t*>(a.rope_sin + (uint32_t)(s * half + m0));
  };
  // The camera rows are per frame (all tokens of a player's frame share one,
  // hub tokens hold zeros), so the camera product of a token is recomputed
  // only when its row differs from the previous token's, with this thread's
  // weights (rows c0.. of [dim][C], packed bf16 pairs) read at that point.
  __syncthreads();   // camera rows staged, red cleared
  if constexpr (C > 0) {
    const int t = threadIdx.x;
    if (t < s_end - s_begin) {
      bool diff = t == 0;
      for (int c = 0; c < CW && !diff; ++c) diff = camw[t * CW + c] != camw[(t - 1) * CW + c];
      cam_new[t] = diff ? 1 : 0;
    }
    __syncthreads();
  }
  float camp[kCPT];   // bf16-rounded camera product of the last new row

  // kTrip tokens per trip (one reduction for all of them); the next trip's
  // projections and RoPE rows are loaded during the current one, into the
  // other of two register sets (no copy between them, so the first use of a
  // set waits only for its own loads, not for the stores and loads issued
  // after them).
  // Past the range's last token a trip repeats it and stores it again.
  struct Pf {
    chw_t x[kTrip];
    rope_t c[kTrip], s[kTrip];
  };
  auto fetch = [&](Pf& f, int s) {
#pragma unroll
    for (int t = 0; t < kTrip; ++t) {
      const int st = min(s + t, s_end - 1);
      f.x[t] = load(st);
      f.c[t] = rc(st);
      f.s[t] = rs(st);
    }
  };
  auto trip = [&](int s, int parity, const Pf& use, Pf& nxt) {
    int sv[kTrip];
    float cpt[kTrip][kCPT];   // camera product of each token of the trip
#pragma unroll
    for (int t = 0; t < kTrip; ++t) sv[t] = min(s + t, s_end - 1);
    // the camera products first: a new row's weight loads then wait only for
    // the previous trip's memory operations, not for this trip's prefetch
    if constexpr (C > 0) {
#pragma unroll
      for (int t = 0; t < kTrip; ++t) {
        const int r = sv[t] - s_begin;
        if (cam_new[r]) {   // workgroup-uniform
          // packed bf16 pairs straight into v_dot2_f32_bf16: weight word w
          // holds elements (e, 2c), (e, 2c+1), camera word c holds cam[2c],
          // cam[2c+1]; the products are exact in fp32 and accumulate in c order
          const u32x4* wr = reinterpret_cast<const u32x4*>(
              (is_k ? a.w_cam_k : a.w_cam_q) + (int64_t)c0 * C);
          const uint32_t* cr = camw + r * CW;
          u32x4 wv[kCPT * CW / 4];
#pragma unroll
          for (int i = 0; i < kCPT * CW / 4; ++i) wv[i] = wr[i];
#pragma unroll
          for (int e = 0; e < kCPT; ++e) {
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < CW; ++c) {
              const int w = e * CW + c;
              // (through a scalar temporary: a bit-cast applied to a vector
              // element subscript directly reads element 0)
              const uint32_t uw = wv[w >> 2][w & 3];
              acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, uw),
                                                    __builtin_bit_cast(bf16x2, cr[c]), acc, false);
            }
            camp[e] = acc;
          }
#pragma unroll
          for (int e = 0; e < kCPT; e += 2) rbf2(camp[e], camp[e + 1]);
        }
#pragma unroll
        for (int e = 0; e < kCPT; ++e) cpt[t][e] = camp[e];
      }
    }
    // unconditional (clamped to the last token past the end), so that the
    // compiler knows exactly which loads are in flight at the first use of `use`
    fetch(nxt, s + kTrip);
    float q[kTrip][kCPT];
#pragma unroll
    for (int t = 0; t < kTrip; ++t)
#pragma unroll
      for (int e = 0; e < kCPT / 2; ++e) {
        q[t][2 * e] = __uint_as_float(use.x[t][e] << 16);
        q[t][2 * e + 1] = __uint_as_float(use.x[t][e] & 0xffff0000u);
      }
    if constexpr (C > 0) {
#pragma unroll
      for (int t = 0; t < kTrip; ++t)
#pragma unroll
        for (int e = 0; e < kCPT; e += 2) {
          q[t][e] += cpt[t][e];
          q[t][e + 1] += cpt[t][e + 1];
          rbf2(q[t][e], q[t][e + 1]);
        }
    }
    float ss[kTrip];
#pragma unroll
    for (int t = 0; t < kTrip; ++t) {
      ss[t] = 0.f;
#pragma unroll
      for (int e = 0; e < kCPT; ++e) ss[t] = fmaf(q[t][e], q[t][e], ss[t]);
    }
    block_sum<kTrip>(ss, red, parity);
#pragma unroll
    for (int t = 0; t < kTrip; ++t) {
      const float inv = __builtin_amdgcn_rsqf(ss[t] * inv_dim + a.eps);
#pragma unroll
      for (int e = 0; e < kCPT; e += 2) {
        q[t][e] *= inv;
        q[t][e + 1] *= inv;
        rbf2(q[t][e], q[t][e + 1]);
        q[t][e] *= g[e];
        q[t][e + 1] *= g[e + 1];
        rbf2(q[t][e], q[t][e + 1]);
      }
      // RoPE on (even, odd) channel pairs of this head
      chw_t qv;
#pragma unroll
      for (int e = 0; e < kCPT / 2; ++e) {
        const float qr = q[t][2 * e] * use.c[t][e] - q[t][2 * e + 1] * use.s[t][e];
        const float qi = q[t][2 * e] * use.s[t][e] + q[t][2 * e + 1] * use.c[t][e];
        qv[e] = f2bf(qr) | (f2bf(qi) << 16);
      }
      const int64_t off = (int64_t)sv[t] * a.out_stride_s + (int64_t)head * a.out_stride_h + d0;
      *reinterpret_cast<chw_t*>(out + off) = qv;
      if (copy_v)
        *reinterpret_cast<chw_t*>(a.v_out + off) =
            *reinterpret_cast<const chw_t*>(a.vx + (uint32_t)(sv[t] * dim + c0));
    }
  };
  // two trips per iteration, the register sets and the reduction buffers
  // alternating
  Pf pa, pb;
  fetch(pa, s_begin);
  for (int s = s_begin; s < s_end; s += 2 * kTrip) {
    trip(s, 0, pa, pb);
    if (s + kTrip < s_end) trip(s + kTrip, 1, pb, pa);
  }
}

// ---- one wave per token (model dims that are multiples of 512) --------------
//
// A wave owns a run of consecutive tokens of one projection and walks it one
// token at a time; lane l holds the NCH 8-channel chunks 8*(64j + l) of the
// token (each chunk of the wave is 1 KB contiguous), so the RMS is one
// register sum and one DPP wave reduction: no LDS and no barrier.  The 8
// channels of a chunk are 4 RoPE pairs of one head, at the same pair index
// 4*(l mod D/8) for every chunk, so a token's cos / sin come in one 16-byte
// load each.  The next token's projection, RoPE rows (and V) are loaded into
// the other of two register sets while the current token is computed.

template <int NCH, bool kCopyV>
struct RowPf {
  u32x4 x[NCH];
  u32x4 v[kCopyV ? NCH : 1];
  float4 c, s;
};

template <int NCH, int C, bool kCopyV>
__global__ __launch_bounds__(256, NCH <= 6 && !kCopyV ? 3 : 2) void row_prologue_kernel(HierPrologueArgs a,
                                                                                     int tpw) {
  constexpr int CW = C > 0 ? C / 2 : 1;      // packed camera words per token
  constexpr int dim = NCH * 512;
  const int lane = threadIdx.x & 63;
  const bool is_k = blockIdx.y != 0;
  const bool copy_v = kCopyV && !is_k;
  const int s_begin = (blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6))) * tpw;
  // RMSNorm gains as fp32, [chunk][half][lane] float4s (conflict-free reads),
  // shared by the workgroup's waves (all of one projection)
  __shared__ float4 g_lds[NCH * 2 * 64];
  for (int i = threadIdx.x; i < NCH * 64; i += blockDim.x) {
    const u32x4 w = *reinterpret_cast<const u32x4*>((is_k ? a.norm_k_w : a.norm_q_w) + 8 * i);
    const int j = i >> 6, l = i & 63;
    g_lds[(2 * j) * 64 + l] = make_float4(__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u),
                                          __uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xffff0000u));
    g_lds[(2 * j + 1) * 64 + l] = make_float4(__uint_as_float(w[2] << 16), __uint_as_float(w[2] & 0xffff0000u),
                                              __uint_as_float(w[3] << 16), __uint_as_float(w[3] & 0xffff0000u));
  }
  __syncthreads();
  if (s_begin >= a.S) return;   // wave-uniform; no barrier follows
  const int s_end = min(a.S, s_begin + tpw);
  const uint16_t* const xin = is_k ? a.kx : a.qx;
  uint16_t* const out = is_k ? a.k_out : a.q_out;
  const int D = a.D, half = D / 2;
  const int d0 = (8 * lane) % D;             // the same in every chunk (D divides 512)
  const int m0 = d0 / 2;
  const float inv_dim = 1.f / (float)dim;
  // output offset of chunk j, token term aside (the launcher runs this kernel
  // only when every output offset fits in 31 bits)
  auto ooff = [&](int j) {
    return (uint32_t)((8 * (64 * j + lane)) / D) * (uint32_t)a.out_stride_h + (uint32_t)d0;
  };
  // element offsets of the [S, dim] projections fit in 32 bits (checked by the launcher)
  auto fetch = [&](RowPf<NCH, kCopyV>& f, int s) {
    const int st = min(s, s_end - 1);
    const uint32_t r0 = (uint32_t)(st * dim + 8 * lane);
    const u32x4* xr = reinterpret_cast<const u32x4*>(xin + r0);
#pragma unroll
    for (int j = 0; j < NCH; ++j) f.x[j] = xr[64 * j];
    if (copy_v) {
      const u32x4* vr = reinterpret_cast<const u32x4*>(a.vx + r0);
#pragma unroll
      for (int j = 0; j < NCH; ++j) f.v[j] = vr[64 * j];
    }
    f.c = *reinterpret_cast<const float4*>(a.rope_cos + (uint32_t)(st * half + m0));
    f.s = *reinterpret_cast<const float4*>(a.rope_sin + (uint32_t)(st * half + m0));
  };
  // camera product of the last camera row seen, bf16-rounded, packed pairs;
  // a token's row is the same for every token of a player's frame (zero for
  // hub tokens), so it is recomputed only where the row changes
  // (in this wave's LDS slot: each lane reads back only what it wrote)
  __shared__ u32x4 camp_lds[C > 0 ? 4 * NCH * 64 : 1];
  u32x4* const camp = camp_lds + (C > 0 ? (s_begin / tpw % 4) * NCH * 64 + lane : 0);
  uint32_t camw_prev[CW] = {};
  auto camera = [&](int s) {
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
        const uint16_t* wbase = is_k ? a.w_cam_k : a.w_cam_q;
        // the weight addresses are formed here, not hoisted out of the token
        // loop (where they would hold 2*NCH registers for a rare branch)
        int ln = lane;
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
          // weight word e*CW + c holds W[cj + e][2c], W[cj + e][2c + 1]; the
          // products are exact in fp32 and accumulate in c order
          const u32x4* wr = reinterpret_cast<const u32x4*>(wbase) + (uint32_t)(64 * j + ln) * (uint32_t)C;
          float pr[8];
#pragma unroll
          for (int hlf = 0; hlf < 2; ++hlf) {   // four channels' weights in registers at a time
            u32x4 wv[CW];
#pragma unroll
            for (int i = 0; i < CW; ++i) wv[i] = wr[hlf * CW + i];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float acc = 0.f;
#pragma unroll
              for (int c = 0; c < CW; ++c) {
                const int w = e * CW + c;
                const uint32_t uw = wv[w >> 2][w & 3];
                acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, uw),
                                                      __builtin_bit_cast(bf16x2, cw[c]), acc, false);
              }
              pr[4 * hlf + e] = acc;
            }
            __builtin_amdgcn_sched_barrier(0);
          }
          u32x4 cp;
#pragma unroll
          for (int e = 0; e < 4; ++e) cp[e] = f2bf(pr[2 * e]) | (f2bf(pr[2 * e + 1]) << 16);
          camp[64 * j] = cp;
        }
      }
    }
  };
  auto token = [&](int s, const RowPf<NCH, kCopyV>& use, RowPf<NCH, kCopyV>& nxt) {
    camera(s);
    // unconditional (clamped to the last token past the end), so that the
    // compiler knows exactly which loads are in flight at the first use of `use`
    fetch(nxt, s + 1);
    // the projection plus the camera product, rounded to bf16 (packed pairs)
    u32x4 qp[NCH];
    float ssp[4] = {0.f, 0.f, 0.f, 0.f};   // sum of squares, four independent chains
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      u32x4 cp;
      if constexpr (C > 0) cp = camp[64 * j];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t u = use.x[j][e];
        if constexpr (C > 0)
          u = pack_bf2(__uint_as_float(u << 16) + __uint_as_float(cp[e] << 16),
                       __uint_as_float(u & 0xffff0000u) + __uint_as_float(cp[e] & 0xffff0000u));
        qp[j][e] = u;
        // bf16 squares are exact in fp32
        ssp[e] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u),
                                                 __builtin_bit_cast(bf16x2, u), ssp[e], false);
      }
    }
    const float ss = wave_sum((ssp[0] + ssp[1]) + (ssp[2] + ssp[3]));
    // unpacked again below rather than kept unpacked (half the registers)
#pragma unroll
    for (int j = 0; j < NCH; ++j) asm volatile("" : "+v"(qp[j]));
    const float inv = __builtin_amdgcn_rsqf(ss * inv_dim + a.eps);
    const float cs[4] = {use.c.x, use.c.y, use.c.z, use.c.w};
    const float sn[4] = {use.s.x, use.s.y, use.s.z, use.s.w};
    const uint32_t srow = (uint32_t)s * (uint32_t)a.out_stride_s;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const float4 ga = g_lds[(2 * j) * 64 + lane], gb = g_lds[(2 * j + 1) * 64 + lane];
      const float gv[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = rbf1(rbf1(__uint_as_float(qp[j][e] << 16) * inv) * gv[2 * e]);
        const float x1 = rbf1(rbf1(__uint_as_float(qp[j][e] & 0xffff0000u) * inv) * gv[2 * e + 1]);
        // RoPE on the (even, odd) pair
        o[e] = pack_bf2(x0 * cs[e] - x1 * sn[e], x0 * sn[e] + x1 * cs[e]);
      }
      const uint32_t off = srow + ooff(j);
      *reinterpret_cast<u32x4*>(out + off) = o;
      if (copy_v) *reinterpret_cast<u32x4*>(a.v_out + off) = use.v[j];
    }
  };
  RowPf<NCH, kCopyV> pa, pb;
  fetch(pa, s_begin);
  for (int s = s_begin; s < s_end; s += 2) {
    token(s, pa, pb);
    if (s + 1 < s_end) token(s + 1, pb, pa);
  }
}

}  // namespace

extern "C" int hier_qkv_prologue(const HierPrologueArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  const HierPrologueArgs& a = *args;
  HIER_REQUIRE(a.S >= 0 && a.H >= 1 && a.H <= 4096 && (a.D == 64 || a.D == 128),
               HIER_EUNSUPPORTED, "prologue supports head_dim 64/128, got H=%d D=%d", a.H, a.D);
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
  HIER_REQUIRE(a.out_stride_s % kCPT == 0 && a.out_stride_h % kCPT == 0 && a.out_stride_s >= 0 &&
                   a.out_stride_h >= 0,
               HIER_EINVAL, "output strides must be non-negative and keep %d-byte alignment",
               2 * kCPT);
  HIER_REQUIRE(hier::span_bytes(a.S, a.out_stride_s, a.out_stride_h, a.H, a.D) <= ((__int128)1 << 48),
               HIER_EUNSUPPORTED, "output view spans more than 2^48 bytes");
  const bool cam = a.cam != nullptr;
  HIER_REQUIRE(!cam || (a.C == 12 && a.w_cam_q && a.w_cam_k), HIER_EUNSUPPORTED,
               "camera adapter supports C=12 with both weights, got C=%d", a.C);
  HIER_REQUIRE(((uintptr_t)a.rope_cos & 15u) == 0 && ((uintptr_t)a.rope_sin & 15u) == 0 &&
                   (!cam || ((uintptr_t)a.cam & 7u) == 0),
               HIER_EINVAL, "RoPE tables must be 16-byte and camera rows 8-byte aligned");
  HIER_REQUIRE((int64_t)a.S * dim <= INT32_MAX, HIER_EUNSUPPORTED,
               "S x model dim must stay below 2^31 elements (got %d x %d)", a.S, dim);
  if (a.S == 0) return HIER_OK;
  const hipStream_t st = (hipStream_t)stream;
  const bool v = a.v_out != nullptr;
  const int nch = dim / 512;
  // the wave kernel forms output offsets in 32 bits
  const int64_t out_ext = (int64_t)(hier::span_bytes(a.S, a.out_stride_s, a.out_stride_h, a.H, a.D) / 2);
  if (dim % 512 == 0 && (nch <= 4 || nch == 6 || nch == 8) && a.out_stride_s % 8 == 0 &&
      a.out_stride_h % 8 == 0 && a.out_stride_s >= 0 && a.out_stride_h >= 0 && out_ext <= INT32_MAX &&
      (!cam || (((uintptr_t)a.w_cam_q | (uintptr_t)a.w_cam_k) & 15u) == 0)) {
    // one wave per run of tpw tokens, about sixteen waves per CU over both projections
    const int tpw = std::max(4, (int)((2ll * a.S + 4095) / 4096));
    const int waves = (a.S + tpw - 1) / tpw;
    const dim3 g2((waves + 3) / 4, 2);
#define HIER_ROW_LAUNCH(N)                                                                        \
  if (nch == N) {                                                                                 \
    if (cam) {                                                                                    \
      if (v) hipLaunchKernelGGL((row_prologue_kernel<N, 12, true>), g2, dim3(256), 0, st, a, tpw);  \
      else hipLaunchKernelGGL((row_prologue_kernel<N, 12, false>), g2, dim3(256), 0, st, a, tpw);   \
    } else {                                                                                      \
      if (v) hipLaunchKernelGGL((row_prologue_kernel<N, 0, true>), g2, dim3(256), 0, st, a, tpw);   \
      else hipLaunchKernelGGL((row_prologue_kernel<N, 0, false>), g2, dim3(256), 0, st, a, tpw);    \
    }                                                                                             \
  }
    HIER_ROW_LAUNCH(1)
    HIER_ROW_LAUNCH(2)
    HIER_ROW_LAUNCH(3)
    HIER_ROW_LAUNCH(4)
    HIER_ROW_LAUNCH(6)
    HIER_ROW_LAUNCH(8)
#undef HIER_ROW_LAUNCH
    return hier::check_launch("row_prologue_kernel");
  }
  const int grid = (a.S + kTokens - 1) / kTokens;
  const int threads = nthr;
  const dim3 g2(grid, 2);
  if (kCPT == 4) {
    if (cam) {
      if (v) hipLaunchKernelGGL((prologue_kernel<12, 4, true>), g2, dim3(threads), 0, st, a);
      else hipLaunchKernelGGL((prologue_kernel<12, 4, false>), g2, dim3(threads), 0, st, a);
    } else {
      if (v) hipLaunchKernelGGL((prologue_kernel<0, 4, true>), g2, dim3(threads), 0, st, a);
      else hipLaunchKernelGGL((prologue_kernel<0, 4, false>), g2, dim3(threads), 0, st, a);
    }
  } else {
    if (cam) {
      if (v) hipLaunchKernelGGL((prologue_kernel<12, 8, true>), g2, dim3(threads), 0, st, a);
      else hipLaunchKernelGGL((prologue_kernel<12, 8, false>), g2, dim3(threads), 0, st, a);
    } else {
      if (v) hipLaunchKernelGGL((prologue_kernel<0, 8, true>), g2, dim3(threads), 0, st, a);
      else hipLaunchKernelGGL((prologue_kernel<0, 8, false>), g2, dim3(threads), 0, st, a);
    }
  }
  return hier::check_launch("prologue_kernel");
}
