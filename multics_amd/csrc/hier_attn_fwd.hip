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
// 64 gathered rows, double buffered; K and V tiles share one row-major layout
// (four threads move one 256-byte key row with 16-byte loads and stores).
//
// Math per wave and tile (v_mfma_f32_32x32x16_bf16):
//   S^T[key, q]  = K[key, :] . Q[q, :]           2 key blocks x D/16 MFMAs
//   online softmax over keys: max / sum are in-register over the lane's 16
//   keys per block plus one swap with lane^32 (v_permlane32_swap)
//   O^T[d, q]   += V^T[d, key] . P^T[key, q]      D/32 x 4 MFMAs
// The P^T operand comes straight from the S^T registers; the matching V^T
// operand is read with ds_read_b64_tr_b16 (a 4 x 16 block of 16-bit values,
// transposed across each 16-lane group), two reads per MFMA.
// fp32 m / l / O, P rounded to bf16 before P.V, exp2 with the log2(e)-scaled
// softmax scale folded into one FMA -- the numerics of the reference kernels
// (hier_tiled_attention.py:112-143).  The running max is refreshed lazily: the
// accumulators are rescaled only when a row's max grows by more than 2^8 in
// exp2 units, which leaves O / l unchanged and keeps P below 256.  Rows with
// no visible key output 0 (hier_segmented_attention.py:104-109).
#include "hier_common.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kKT = 64;                // keys per LDS tile
constexpr float kRescaleLog2 = 8.0f;   // lazy-rescale threshold (exp2 units)

// LDS row pitches (bf16).  K rows are read 16 rows per cycle at one column
// (the S^T A operand): consecutive rows shift by 4 banks.  V rows are read
// four keys x four 8-byte chunks per 16-lane group (transposed reads) and are
// written eight keys x two adjacent 16-byte chunks per group: consecutive rows
// shift by 8 (D=128) or 40 (D=64) banks.  All three patterns are free of bank
// conflicts on a 64-bank LDS.
template <int D>
struct Tile {
  static constexpr int kPitchK = D == 128 ? 136 : 72;
  static constexpr int kPitchV = D == 128 ? 144 : 80;
};

template <int D>
struct Smem {
  uint16_t k[2][kKT * Tile<D>::kPitchK];
  uint16_t v[2][kKT * Tile<D>::kPitchV];
  uint32_t km[2][kKT];
};

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

// V^T operand of O^T += V^T P^T for rows d = d0 + (lane & 15) of this lane's
// 16-lane group: two transposed reads of 4 keys each (keys 16kc + 4h + r and
// 16kc + 8 + 4h + r, r = 0..3, h = lane >> 5) -- the key order of the P^T
// operand taken from the S^T accumulator.
template <int KP>
__device__ __forceinline__ bf16x8 load_vt(const uint16_t* vbuf, int kc, int d0, int lane) {
  const int h = lane >> 5, i = lane & 15;
  const int key = 16 * kc + 4 * h + (i >> 2);
  const uint16_t* p0 = vbuf + key * KP + d0 + 4 * (i & 3);
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p0);
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0 + 8 * KP));
  const s16x8 ab = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, ab);
}

template <int D>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(HierFwdArgs a, int total) {
  constexpr int NC = D / 16;   // d-chunks of QK^T
  constexpr int NDB = D / 32;  // d-blocks of O^T
  constexpr int KPK = Tile<D>::kPitchK;
  constexpr int KPV = Tile<D>::kPitchV;
  constexpr int NV = D / 32;   // 16-byte vectors per thread per K (or V) tile
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

  // loaders (every thread moves NV 16-byte vectors of K and of V per tile):
  //  K: key = tid % 64, elements [q*D/4, (q+1)*D/4) with q = tid / 64
  //  V: 16-lane group m = tid / 16 stores keys 8*(m%8) + i/2 (i = tid % 16),
  //     16-byte chunk 2*((m/8)*NV + e) + i%2 for vector e
  const int kkey = tid & 63, kq = tid >> 6;
  const int vgrp = tid >> 4, vi = tid & 15;
  const int vkey = 8 * (vgrp & 7) + (vi >> 1);
  const int64_t k_head = (int64_t)head * a.k_sh, v_head = (int64_t)head * a.v_sh;
  u32x4 kreg[NV], vreg[NV];
  uint32_t mreg = 0;
  const int ntiles = kv_cnt / kKT;
  int kidx = 0, vidx = 0;   // K/V pool rows of the next tile to fetch

  auto fetch_idx = [&](int t) {   // t < ntiles
    const int base = kv_off + t * kKT;
    kidx = a.tile_kv_idx[base + kkey];
    vidx = a.tile_kv_idx[base + vkey];
  };
  auto gload = [&](int t) {       // uses kidx / vidx fetched for tile t
    const uint16_t* kp = a.k + (int64_t)kidx * a.k_ss + k_head + kq * (D / 4);
    const uint16_t* vp = a.v + (int64_t)vidx * a.v_ss + v_head;
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      kreg[e] = *reinterpret_cast<const u32x4*>(kp + 8 * e);
      const int chunk = 2 * ((vgrp >> 3) * NV + e) + (vi & 1);
      vreg[e] = *reinterpret_cast<const u32x4*>(vp + 8 * chunk);
    }
    if (tid < kKT) mreg = a.tile_kv_mask[kv_off + t * kKT + tid];
  };
  auto lstore = [&](int buf) {
    uint16_t* kd = &sm.k[buf][kkey * KPK + kq * (D / 4)];
    uint16_t* vd = &sm.v[buf][vkey * KPV];
#pragma unroll
    for (int e = 0; e < NV; ++e) {
      *reinterpret_cast<u32x4*>(kd + 8 * e) = kreg[e];
      const int chunk = 2 * ((vgrp >> 3) * NV + e) + (vi & 1);
      *reinterpret_cast<u32x4*>(vd + 8 * chunk) = vreg[e];
    }
    if (tid < kKT) sm.km[buf][tid] = mreg;
  };

  const float c2 = a.scale * 1.4426950408889634f;  // softmax scale * log2(e)
  const float thr = kRescaleLog2 / c2;             // lazy-rescale margin in score units
  float m_ref = -INFINITY, l_run = 0.f;
  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
  const f32x16 zero = {};

  if (ntiles > 0) {
    fetch_idx(0);
    gload(0);
    lstore(0);
    fetch_idx(ntiles > 1 ? 1 : 0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    // Prefetch tile t+1 unconditionally (the last iteration re-reads tile t):
    // a conditional load here makes the compiler wait on it before the MFMAs.
    const int tn = t + 1 < ntiles ? t + 1 : t;
    gload(tn);
    fetch_idx(t + 2 < ntiles ? t + 2 : tn);
    if (wave_active) {
      // ---- S^T = K Q^T -------------------------------------------------------
      f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const uint16_t* kp = &sm.k[buf][(kb * 32 + col) * KPK + 8 * half];
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            *reinterpret_cast<const bf16x8*>(kp), qf[0], zero, 0, 0, 0);
#pragma unroll
        for (int c = 1; c < NC; ++c) {
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
      // ---- online softmax (lazy rescale) ----------------------------------------
      float mx = fmaxf(s[0][0], s[0][1]);
#pragma unroll
      for (int r = 2; r < 16; r += 2) mx = fmaxf(mx, fmaxf(s[0][r], s[0][r + 1]));
#pragma unroll
      for (int r = 0; r < 16; r += 2) mx = fmaxf(mx, fmaxf(s[1][r], s[1][r + 1]));
      mx = pair_max(mx);
      if (__ballot(mx > m_ref + thr) != 0) {
        const float m_new = fmaxf(m_ref, mx);
        const float alpha = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f((m_ref - m_new) * c2);
        m_ref = m_new;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      }
      const float nb = (m_ref == -INFINITY) ? 0.f : -m_ref * c2;
      float ps0 = 0.f, ps1 = 0.f;
      bf16x8 pk[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(fmaf(s[kb][r], c2, nb));
          if (r & 1) ps1 += p; else ps0 += p;
          pk[kb * 2 + (r >> 3)][r & 7] = (__bf16)p;
        }
      l_run += ps0 + ps1;
      // ---- O^T += V^T P^T ------------------------------------------------------
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int d0 = db * 32 + 16 * ((lane >> 4) & 1);
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
          const bf16x8 vf = load_vt<KPV>(sm.v[buf], kc, d0, lane);
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
      const float lse = l_tot > 0.f ? m_ref * a.scale + __logf(l_tot) : -INFINITY;
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
