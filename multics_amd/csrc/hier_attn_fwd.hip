// Block-sparse, frame-causal flash-attention forward for gfx950 (CDNA4).
//
// Work item = up to 128 query rows of one stream (a player, a local-hub slot or
// the global hub) of one temporal block, for one head.  The rows attend to the
// stream's key list (the ordered union over the block's query frames of the
// reference's per-frame key lists, hier_segmented_attention.py:276-368) with a
// per-key bitmask saying which query frames may see it.  Only listed keys are
// visited; there is no dense S x S mask anywhere.
//
// Per workgroup: 4 waves x 32 query rows.  Keys stream through LDS in tiles of
// 64 gathered rows, double buffered: K row-major, V transposed (d-major) with
// the keys of every 16-key group permuted so that the P operand of P.V can be
// fed straight from the registers of the QK^T result.
//
// Math per wave and tile (v_mfma_f32_32x32x16_bf16):
//   S^T[key, q]  = K[key, :] . Q[q, :]           2 key blocks x D/16 MFMAs
//   online softmax over keys: max / sum are in-register over the lane's 16
//   keys per block plus one swap with lane^32 (v_permlane32_swap)
//   O^T[d, q]   += V^T[d, key] . P^T[key, q]      D/32 x 4 MFMAs
// fp32 m / l / O, P rounded to bf16 before P.V, exp2 with the log2(e)-scaled
// softmax scale folded into one FMA -- the numerics of the reference kernels
// (hier_tiled_attention.py:112-143).  Rows with no visible key output 0
// (hier_segmented_attention.py:104-109).
#include "hier_common.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kRows = 32 * kWaves;     // query rows per work item
constexpr int kKT = 64;                // keys per LDS tile
constexpr int kVPitch = kKT + 8;       // bf16 per V^T row (padded)

template <int D>
struct Smem {
  static constexpr int kPitch = D + 8;             // bf16 per K row (padded)
  uint16_t k[2][kKT * kPitch];
  uint16_t vt[2][D * kVPitch];
  uint32_t km[2][kKT];
};

// Position of key x (0..15) of a 16-key group inside a V^T row: the 8 keys that
// one half-wave multiplies in P.V become contiguous (a 16-byte LDS read).
__device__ __forceinline__ int vt_pos(int x) {
  return ((x >> 2) & 1) * 8 + (x >> 3) * 4 + (x & 3);
}

__device__ __forceinline__ float pair_max(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) v |= __shfl_xor(v, d, 64);
  return v;
}

__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);  // round to nearest even
}

template <int D>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(HierFwdArgs a, int total) {
  constexpr int NC = D / 16;   // d-chunks of QK^T
  constexpr int NDB = D / 32;  // d-blocks of O^T
  constexpr int KP = Smem<D>::kPitch;
  __shared__ __align__(16) Smem<D> sm;

  // XCD-aware mapping: consecutive logical items land on the same XCD (the
  // dispatcher round-robins workgroups over 8 XCDs), so the items sharing a
  // head and overlapping key windows share one L2.
  const int G = gridDim.x;
  const int bid = blockIdx.x;
  const int logical = (bid & 7) * (G >> 3) + (bid >> 3);
  if (logical >= total) return;
  const int head = logical / a.n_items;
  const int item = logical - head * a.n_items;

  const int32_t* it = a.tile_items + (int64_t)item * 8;
  const int qbase = it[0], qstride = it[1], qlen = it[2];
  const int row_start = it[3], row_count = it[4];
  const int kv_off = it[5], kv_cnt = it[6];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, col = lane & 31;

  // this lane's query row
  const int rrel = wave * 32 + col;
  const bool valid = rrel < row_count;
  const int ri = row_start + (valid ? rrel : 0);
  const int qframe = ri / qlen;
  const int qtok = qbase + qframe * qstride + (ri - qframe * qlen);
  const bool wave_active = wave * 32 < row_count;
  const uint32_t wave_bits = wave_or(valid ? (1u << qframe) : 0u);

  // Q fragments (B operand of S^T = K Q^T): row qtok, d = 16c + 8*half + [0,8)
  bf16x8 qf[NC];
  {
    const uint16_t* qp = a.q + (int64_t)qtok * a.q_ss + (int64_t)head * a.q_sh + 8 * half;
#pragma unroll
    for (int c = 0; c < NC; ++c) qf[c] = *reinterpret_cast<const bf16x8*>(qp + 16 * c);
  }

  // loader mapping: 32 key pairs x 8 d-groups; thread (pair, dg) moves keys
  // 2*pair and 2*pair+1, elements [dg*D/8, (dg+1)*D/8)
  constexpr int DG = D / 8;              // elements per d-group
  constexpr int NV = DG / 8;             // 16-byte vectors per key per thread
  const int pair = tid & 31, dg = tid >> 5;
  const int64_t k_head = (int64_t)head * a.k_sh, v_head = (int64_t)head * a.v_sh;

  u32x4 kreg[2][NV], vreg[2][NV];
  uint32_t mreg = 0;
  const int ntiles = kv_cnt / kKT;

  auto gload = [&](int t) {
    const int base = kv_off + t * kKT;
    const int i0 = a.tile_kv_idx[base + 2 * pair];
    const int i1 = a.tile_kv_idx[base + 2 * pair + 1];
    const uint16_t* k0 = a.k + (int64_t)i0 * a.k_ss + k_head + dg * DG;
    const uint16_t* k1 = a.k + (int64_t)i1 * a.k_ss + k_head + dg * DG;
    const uint16_t* v0 = a.v + (int64_t)i0 * a.v_ss + v_head + dg * DG;
    const uint16_t* v1 = a.v + (int64_t)i1 * a.v_ss + v_head + dg * DG;
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      kreg[0][e] = *reinterpret_cast<const u32x4*>(k0 + 8 * e);
      kreg[1][e] = *reinterpret_cast<const u32x4*>(k1 + 8 * e);
      vreg[0][e] = *reinterpret_cast<const u32x4*>(v0 + 8 * e);
      vreg[1][e] = *reinterpret_cast<const u32x4*>(v1 + 8 * e);
    }
    if (tid < kKT) mreg = a.tile_kv_mask[base + tid];
  };

  auto lstore = [&](int buf) {
    const int key0 = 2 * pair;
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      *reinterpret_cast<u32x4*>(&sm.k[buf][key0 * KP + dg * DG + 8 * e]) = kreg[0][e];
      *reinterpret_cast<u32x4*>(&sm.k[buf][(key0 + 1) * KP + dg * DG + 8 * e]) = kreg[1][e];
    }
    // V^T: word (keys key0, key0+1) of row d; key0 even so both share a word
    const int pos = (key0 & ~15) + vt_pos(key0 & 15);
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      const u32x4 w0 = vreg[0][e], w1 = vreg[1][e];
#pragma unroll
      for (int h2 = 0; h2 < 4; ++h2) {
        const int d = dg * DG + 8 * e + 2 * h2;
        const uint32_t lo = (w0[h2] & 0xffffu) | (w1[h2] << 16);
        const uint32_t hi = (w0[h2] >> 16) | (w1[h2] & 0xffff0000u);
        *reinterpret_cast<uint32_t*>(&sm.vt[buf][d * kVPitch + pos]) = lo;
        *reinterpret_cast<uint32_t*>(&sm.vt[buf][(d + 1) * kVPitch + pos]) = hi;
      }
    }
    if (tid < kKT) sm.km[buf][tid] = mreg;
  };

  const float c2 = a.scale * 1.4426950408889634f;  // softmax scale * log2(e)
  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;

  if (ntiles > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) gload(t + 1);
    if (wave_active) {
      // ---- S^T = K Q^T -------------------------------------------------------
      f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
        const uint16_t* kp = &sm.k[buf][(kb * 32 + col) * KP + 8 * half];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          bf16x8 kf = *reinterpret_cast<const bf16x8*>(kp + 16 * c);
          s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[c], s[kb], 0, 0, 0);
        }
      }
      // ---- visibility ---------------------------------------------------------
      const uint32_t blk = a.tile_blk_and[kv_off / kKT + t];
      if ((blk & wave_bits) != wave_bits) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const u32x4 mk = *reinterpret_cast<const u32x4*>(&sm.km[buf][kb * 32 + 8 * g4 + 4 * half]);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (!((mk[e] >> qframe) & 1u)) s[kb][4 * g4 + e] = -INFINITY;
          }
      }
      // ---- online softmax -----------------------------------------------------
      float mx = s[0][0];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
      mx = pair_max(mx);
      const float m_new = fmaxf(m_run, mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * c2);
      const float nb = -m_use * c2;
      m_run = m_new;
      float psum = 0.f;
      bf16x8 pk[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(fmaf(s[kb][r], c2, nb));
          psum += p;
          pk[kb * 2 + (r >> 3)][r & 7] = (__bf16)p;
        }
      l_run = l_run * alpha + psum;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      // ---- O^T += V^T P^T ------------------------------------------------------
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const uint16_t* vp = &sm.vt[buf][(db * 32 + col) * kVPitch + 8 * half];
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
          bf16x8 vf = *reinterpret_cast<const bf16x8*>(vp + 16 * kc);
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pk[kc], o[db], 0, 0, 0);
        }
      }
    }
    if (t + 1 < ntiles) lstore(buf ^ 1);
    __syncthreads();
  }

  if (!wave_active) return;
  const float l_tot = pair_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (valid) {
    uint16_t* op = a.o + (int64_t)qtok * a.o_ss + (int64_t)head * a.o_sh;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = db * 32 + 8 * g4 + 4 * half;
        u32x2 w;
        w[0] = (uint32_t)f2bf(o[db][4 * g4 + 0] * inv) | ((uint32_t)f2bf(o[db][4 * g4 + 1] * inv) << 16);
        w[1] = (uint32_t)f2bf(o[db][4 * g4 + 2] * inv) | ((uint32_t)f2bf(o[db][4 * g4 + 3] * inv) << 16);
        *reinterpret_cast<u32x2*>(op + d0) = w;
      }
    if (a.lse && half == 0) {
      const float lse = l_tot > 0.f ? m_run * a.scale + __logf(l_tot) : -INFINITY;
      a.lse[(int64_t)head * a.lse_stride_h + qtok] = lse;
    }
  }
}

}  // namespace

extern "C" int hier_attn_fwd(const HierFwdArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  const HierFwdArgs& a = *args;
  HIER_REQUIRE(a.D == 128 || a.D == 64, HIER_EUNSUPPORTED, "head_dim must be 64 or 128, got %d", a.D);
  HIER_REQUIRE(a.H >= 1 && a.n_items >= 0, HIER_EINVAL, "invalid H=%d n_items=%d", a.H, a.n_items);
  HIER_REQUIRE(a.q && a.k && a.v && a.o && a.tile_items && a.tile_kv_idx && a.tile_kv_mask &&
                   a.tile_blk_and,
               HIER_EINVAL, "NULL tensor pointer");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  HIER_REQUIRE(al16(a.q) && al16(a.k) && al16(a.v) && al16(a.o), HIER_EINVAL,
               "q/k/v/o must be 16-byte aligned");
  HIER_REQUIRE(a.q_ss % 8 == 0 && a.q_sh % 8 == 0 && a.k_ss % 8 == 0 && a.k_sh % 8 == 0 &&
                   a.v_ss % 8 == 0 && a.v_sh % 8 == 0 && a.o_ss % 4 == 0 && a.o_sh % 4 == 0,
               HIER_EINVAL, "strides must keep 16-byte rows aligned");
  if (a.n_items == 0) return HIER_OK;
  const int64_t total = (int64_t)a.n_items * a.H;
  HIER_REQUIRE(total < (1ll << 31) - 8, HIER_EUNSUPPORTED, "too many work items");
  const int grid = (int)((total + 7) / 8 * 8);
  if (a.D == 128)
    hipLaunchKernelGGL(attn_fwd_kernel<128>, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, a,
                       (int)total);
  else
    hipLaunchKernelGGL(attn_fwd_kernel<64>, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, a,
                       (int)total);
  return hier::check_launch("attn_fwd_kernel");
}
