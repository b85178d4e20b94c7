// Backward of the block-sparse frame-causal attention for gfx950 (CDNA4).
//
// With P = exp(scale * Q K^T - lse) (lse from the forward), dP = dO V^T,
// delta = rowsum(dO * O) and dS = P * (dP - delta):
//   dQ = scale * dS K,   dK = scale * dS^T Q,   dV = P^T dO.
// Two kernels, each writing every gradient row from exactly one workgroup
// (deterministic, no global atomics):
//
// dq_kernel   query-major, over the forward tile list (128 query rows per
//             item, 4 waves x 32).  Per 32-key block:
//               S^T  = K Q^T          (K rows from LDS, Q^T in registers)
//               dP^T = V dO^T         (V rows from LDS, dO^T in registers)
//               dS^T = P^T (dP^T - delta)
//               dQ^T += K^T dS^T      (K transposed out of LDS)
//             Also writes -delta and lse2 = lse * log2(e) per query row.
// dkv_kernel  key-major, over the transposed tile list (128 key rows per
//             item, lists of query rows with a bitmask over key frames),
//             eight waves: wave w and wave w+4 own the same 32 key rows (one
//             wave cannot hold both accumulators at two waves per SIMD).
//             Per 64-query tile:
//               wave w:   S = Q K^T, P;  P to LDS;  dV^T += dO^T P
//               wave w+4: dP - delta = dO V^T accumulated onto -delta;
//                         dS = P (dP - delta);  dK^T += Q^T dS
//             (Q / dO rows from LDS, K^T / V^T in registers, Q / dO
//             transposed out of LDS for the accumulations), with the S / dP
//             products of tile t+1 overlapping the accumulations of tile t.
// The lane layouts are the forward's: an MFMA result keeps one column per
// lane and its rows {8*(r/4) + 4*(lane/32) + r%4}, which is exactly the
// permuted k order of the next MFMA's register operand, so P and dS go from
// the accumulators to bf16 operands without any shuffle.  Tiles are copied
// with global_load_lds_dwordx4 into the swizzled layouts of hier_tile.h.
//
// Membership STE: with tile_kv_class set, dq_kernel also sums the fp32 dS
// of each row's membership-gated keys per class (dq_kernel<D, true>);
// ste_kernel does the same over a separate list of the gated keys only.
#include "hier_common.h"
#include "hier_launch.h"
#include "hier_tile.h"

#include <algorithm>
#include <type_traits>
#include <mutex>

namespace {

using namespace hier::tile;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr float kLog2e = 1.4426950408889634f;

// ---- shared helpers --------------------------------------------------------

template <int D>
__device__ __forceinline__ void load_row(bf16x8* dst, const uint16_t* row, int lane) {
  const uint16_t* p = row + 8 * (lane >> 5);
#pragma unroll
  for (int c = 0; c < Geo<D>::NC; ++c) dst[c] = *reinterpret_cast<const bf16x8*>(p + 16 * c);
}

template <int D>
__device__ __forceinline__ f32x16 row_mfma(const bf16x8* b, const char* tile, const int* off,
                                           int blk) {
  const char* base = tile + blk * 32 * Geo<D>::ROWB;
  const f32x16 zero = {};
  f32x16 s = mfma(*reinterpret_cast<const bf16x8*>(base + off[0]), b[0], zero);
#pragma unroll
  for (int c = 1; c < Geo<D>::NC; ++c)
    s = mfma(*reinterpret_cast<const bf16x8*>(base + off[c]), b[c], s);
  return s;
}

template <int D>
__device__ __forceinline__ f32x16 row_mfma_from(f32x16 s, const bf16x8* b, const char* tile,
                                                const int* off, int blk) {
  const char* base = tile + blk * 32 * Geo<D>::ROWB;
#pragma unroll
  for (int c = 0; c < Geo<D>::NC; ++c)
    s = mfma(*reinterpret_cast<const bf16x8*>(base + off[c]), b[c], s);
  return s;
}

// acc[db] += A^T(block rows 32*blk .. +32, d-block db) . p[j] over the two
// 16-row chunks j of the block; A is read transposed from a kBothRead tile.
template <int D>
__device__ __forceinline__ void tr_mfma(f32x16* acc, const bf16x8* p, const char* tile,
                                        const int (*tr)[2], int blk) {
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int db = 0; db < Geo<D>::NDB; ++db) {
      const char* base = tile + (2 * blk + j) * 16 * Geo<D>::ROWB;
      acc[db] = mfma(tr_read(base + tr[db][0], base + tr[db][1]), p[j], acc[db]);
    }
}

template <int D>
__device__ __forceinline__ void store_acc(uint16_t* row, const f32x16* acc, float mul, int lane) {
  const int half = lane >> 5;
#pragma unroll
  for (int db = 0; db < Geo<D>::NDB; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d0 = db * 32 + 8 * g4 + 4 * half;
      u32x2 w;
      w[0] = (uint32_t)f2bf(acc[db][4 * g4 + 0] * mul) | ((uint32_t)f2bf(acc[db][4 * g4 + 1] * mul) << 16);
      w[1] = (uint32_t)f2bf(acc[db][4 * g4 + 2] * mul) | ((uint32_t)f2bf(acc[db][4 * g4 + 3] * mul) << 16);
      *reinterpret_cast<u32x2*>(row + d0) = w;
    }
}

__device__ __forceinline__ uint32_t keep_mask(uint32_t bits, int bit) {
  return (uint32_t)__builtin_amdgcn_sbfe((int)bits, bit, 1);   // 0 or ~0
}

// ---- membership STE sums -----------------------------------------------------

constexpr int kSteClasses = 16;
constexpr int kSteSlots = kWaves * 32;   // one slot per (class, query row of a workgroup)

// Adds a lane's 16 dS terms of one 32-key block into the slots of their
// classes, acc[class * kSteSlots]; a class outside [0, kSteClasses) marks a
// key whose edge no membership bit gates, and is skipped.  The keys of a
// block mostly share one class (lists keep each class's keys together): a
// lane whose 16 keys do adds their sum once, otherwise each term.  Only the
// two lanes of a query row (its two key halves) share a slot.
__device__ __forceinline__ void ste_add(float* acc, const float* ds, const uint32_t* cls,
                                        bool valid) {
  bool same = true;
#pragma unroll
  for (int i = 1; i < 16; ++i) same = same && cls[i] == cls[0];
  if (!valid) return;
  if (same) {
    if (cls[0] < kSteClasses) {
      float t = ds[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) t += ds[i];
      atomicAdd(&acc[cls[0] * kSteSlots], t);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (cls[i] < kSteClasses) atomicAdd(&acc[cls[i] * kSteSlots], ds[i]);
  }
}

// ---- dQ (query-major) --------------------------------------------------------

// LDS stages: K[2] (rows and transposed) | V[2] (rows) | masks[2] | STE
// classes[2] (membership STE only), each its own __shared__ array.  Distinct
// arrays let the compiler see that the copies into one stage never alias the
// reads of the other; given one array it waits for every outstanding copy
// before the first LDS read that follows them.
struct QStages {
  char* k[2];
  char* v[2];
  char* m[2];
  char* c[2];
};

template <int D>
struct QCtx {
  const HierBwdArgs* a;
  const char* gk;
  const char* gv;
  const int32_t* kv_idx;
  const uint32_t* kv_mask;
  const int32_t* kv_cls;       // STE class of each list entry (membership STE only)
  float* ste;                  // the lane's row's STE slots, ste[class * kSteSlots]
  int t1;                      // first tile with a gated key (membership STE only)
  uint32_t k_ss_b, v_ss_b;
  float c2;
  int nt, wave, lane;
  bool active;
  Copier<D, kBothRead> ck;     // K and V tiles share one layout (rows + transposed reads)
  int krow[Geo<D>::NC], ktr[Geo<D>::NDB][2];
  // rows
  bf16x8 q[Geo<D>::NC], dov[Geo<D>::NC];
  f32x16 dq[Geo<D>::NDB];
  float lse2, delta;
  int qtok, qframe;
  bool valid;
};

// Scheduling pattern of one phase: N x (one MFMA, R LDS reads, V VALU
// instructions), four LDS reads issued ahead.  The compiler's own schedule
// clusters MFMAs and VALU work; this interleaves them so that the VALU work
// of one block runs under the MFMAs of the next.  (Same box, C5 backward:
// 2.79 ms unscheduled, 2.77 with two reads ahead, 2.70-2.72 with four or
// six, 2.81 with eight.)
template <int N, int R, int V>
__device__ __forceinline__ void sched_phase() {
  __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, R, 0);
    if (V > 0) __builtin_amdgcn_sched_group_barrier(0x002, V, 0);
  }
}

// P = exp2(S c2 - lse2) of one 32-key block, in place.
__device__ __forceinline__ void p_exp(f32x16& s, float c2, float lse2) {
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] = __builtin_amdgcn_exp2f(fmaf(s[i], c2, -lse2));
}

// dS^T = P^T (dP^T - delta) of block kb, the keys the lane's query frame may
// not see zeroed, rounded to the bf16 operand of the dQ product.  With STE,
// the fp32 dS of the block's gated keys (class words `cl`, from LDS) is also
// added into the row's class slots.
template <bool STE>
__device__ __forceinline__ void ds_block(const f32x16& p, const f32x16& dp, float delta,
                                         const uint32_t* mk, const uint32_t* cl, float* ste,
                                         bool valid, int kb, int qframe, int lane, bf16x8* dsb) {
  float ds[16];
  uint32_t cls[16];
#pragma unroll
  for (int g4 = 0; g4 < 4; ++g4) {
    const int k0 = kb * 32 + 8 * g4 + 4 * (lane >> 5);
    const u32x4 w = *reinterpret_cast<const u32x4*>(&mk[k0]);
    if constexpr (STE) {
      const u32x4 c4 = *reinterpret_cast<const u32x4*>(&cl[k0]);
#pragma unroll
      for (int e = 0; e < 4; ++e) cls[4 * g4 + e] = c4[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 4 * g4 + e;
      ds[i] = __uint_as_float(__float_as_uint(p[i] * (dp[i] - delta)) & keep_mask(w[e], qframe));
      dsb[i >> 3][i & 7] = (__bf16)ds[i];
    }
  }
  if constexpr (STE) ste_add(ste, ds, cls, valid);
}

// Tile t: works on stage PAR while tile t+1 is copied into stage PAR^1 in two
// bursts, K (with the masks) before the first 32-key block and V before the
// second, and loads the key indices of tile t+2.  Every global load is
// waited for with the copies at the end, so nothing in the MFMA work waits on
// the copies in flight.  The two blocks are software-pipelined so that each
// group of eight MFMAs has independent VALU work beside it:
//     S(0) ; dP(0) || exp S(0) ; [V copy] ; S(1) || dS(0) ;
//     dP(1) || exp S(1) ; dQ(0) || dS(1) ; dQ(1)
// (the masks are applied to every block: 16 ANDs under the MFMAs are cheaper
// than a branch, which would split the schedule).
// STE: a tile before the first one with a gated key (dq_tile_ste handles
// those); the last such tile copies the class words of the next.
template <int D, int PAR, bool STE>
__device__ __forceinline__ void dq_tile(QCtx<D>& c, int t, Idx<D>& inext, const QStages& st) {
  const bool more = t + 1 < c.nt;
  if (more) {
    copy_tile<D, kBothRead>(c.gk, c.k_ss_b, c.ck, inext, st.k[PAR ^ 1], c.wave);
    copy_dwords(c.kv_mask + (t + 1) * kSlab, st.m[PAR ^ 1], c.lane);
    if (STE && t + 1 == c.t1) copy_dwords(c.kv_cls + (t + 1) * kSlab, st.c[PAR ^ 1], c.lane);
  }
  const char* ks = st.k[PAR];
  const char* vs = st.v[PAR];
  const uint32_t* mk = reinterpret_cast<const uint32_t*>(st.m[PAR]);
  constexpr int NC = Geo<D>::NC, NDB = Geo<D>::NDB;
  f32x16 s0, dp0;
  if (c.active) {
    s0 = row_mfma<D>(c.q, ks, c.krow, 0);
    dp0 = row_mfma<D>(c.dov, vs, c.krow, 0);
    p_exp(s0, c.c2, c.lse2);
    // S(0): MFMAs with their operand reads; dP(0) with the exps of S(0)
    sched_phase<NC, 1, 0>();
    sched_phase<NC, 1, 4>();
  }
  if (more) {
    copy_tile<D, kBothRead>(c.gv, c.v_ss_b, c.ck, inext, st.v[PAR ^ 1], c.wave);
    inext = load_idx<D>(c.kv_idx, min(t + 2, c.nt - 1), c.ck.idx_off);
  }
  if (c.active) {
    f32x16 s1 = row_mfma<D>(c.q, ks, c.krow, 1);
    bf16x8 ds0[2], ds1[2];
    ds_block<false>(s0, dp0, c.delta, mk, nullptr, nullptr, false, 0, c.qframe, c.lane, ds0);
    const f32x16 dp1 = row_mfma<D>(c.dov, vs, c.krow, 1);
    p_exp(s1, c.c2, c.lse2);
    tr_mfma<D>(c.dq, ds0, ks, c.ktr, 0);
    ds_block<false>(s1, dp1, c.delta, mk, nullptr, nullptr, false, 1, c.qframe, c.lane, ds1);
    tr_mfma<D>(c.dq, ds1, ks, c.ktr, 1);
    // S(1) || dS(0); dP(1) || exp S(1); dQ(0) || dS(1); dQ(1)
    sched_phase<NC, 1, 7>();
    sched_phase<NC, 1, 4>();
    sched_phase<2 * NDB, 2, 7>();
    sched_phase<2 * NDB, 2, 0>();
  }
  wait_copies();
  __syncthreads();
}

// A tile with a gated key (membership STE): the same copies and products, the
// two 32-key blocks one after the other (fewer values live than in the
// pipelined dq_tile, which leaves room for the per-class sums of dS).
template <int D, int PAR>
__device__ __forceinline__ void dq_tile_ste(QCtx<D>& c, int t, Idx<D>& inext,
                                            const QStages& st) {
  const bool more = t + 1 < c.nt;
  if (more) {
    copy_tile<D, kBothRead>(c.gk, c.k_ss_b, c.ck, inext, st.k[PAR ^ 1], c.wave);
    copy_dwords(c.kv_mask + (t + 1) * kSlab, st.m[PAR ^ 1], c.lane);
    copy_dwords(c.kv_cls + (t + 1) * kSlab, st.c[PAR ^ 1], c.lane);
  }
  const char* ks = st.k[PAR];
  const char* vs = st.v[PAR];
  const uint32_t* mk = reinterpret_cast<const uint32_t*>(st.m[PAR]);
  const uint32_t* cl = reinterpret_cast<const uint32_t*>(st.c[PAR]);
  auto block = [&](int kb) {
    f32x16 s = row_mfma<D>(c.q, ks, c.krow, kb);
    const f32x16 dp = row_mfma<D>(c.dov, vs, c.krow, kb);
    p_exp(s, c.c2, c.lse2);
    bf16x8 ds[2];
    ds_block<true>(s, dp, c.delta, mk, cl, c.ste, c.valid, kb, c.qframe, c.lane, ds);
    tr_mfma<D>(c.dq, ds, ks, c.ktr, kb);
  };
  if (c.active) block(0);
  if (more) {
    copy_tile<D, kBothRead>(c.gv, c.v_ss_b, c.ck, inext, st.v[PAR ^ 1], c.wave);
    inext = load_idx<D>(c.kv_idx, min(t + 2, c.nt - 1), c.ck.idx_off);
  }
  if (c.active) block(1);
  wait_copies();
  __syncthreads();
}

// Tile t of an item of at most 32 rows: waves 0 and 1 hold the same rows and
// take one 32-key block each (wave w: block w), so such an item -- a hub
// stream's rows, a player block's ragged last item -- runs on two waves
// instead of one; waves 2 and 3 only copy.  The two waves' dQ and STE sums
// are added at the end.
template <int D, int PAR, bool STE>
__device__ __forceinline__ void dq_tile_split(QCtx<D>& c, int t, Idx<D>& inext,
                                              const QStages& st) {
  if (t + 1 < c.nt) {
    copy_tile<D, kBothRead>(c.gk, c.k_ss_b, c.ck, inext, st.k[PAR ^ 1], c.wave);
    copy_dwords(c.kv_mask + (t + 1) * kSlab, st.m[PAR ^ 1], c.lane);
    if (STE && t + 1 >= c.t1) copy_dwords(c.kv_cls + (t + 1) * kSlab, st.c[PAR ^ 1], c.lane);
    copy_tile<D, kBothRead>(c.gv, c.v_ss_b, c.ck, inext, st.v[PAR ^ 1], c.wave);
    inext = load_idx<D>(c.kv_idx, min(t + 2, c.nt - 1), c.ck.idx_off);
  }
  if (c.active) {
    const int kb = c.wave;
    const char* ks = st.k[PAR];
    const uint32_t* mk = reinterpret_cast<const uint32_t*>(st.m[PAR]);
    f32x16 s = row_mfma<D>(c.q, ks, c.krow, kb);
    const f32x16 dp = row_mfma<D>(c.dov, st.v[PAR], c.krow, kb);
    p_exp(s, c.c2, c.lse2);
    bf16x8 ds[2];
    if (STE && t >= c.t1)
      ds_block<true>(s, dp, c.delta, mk, reinterpret_cast<const uint32_t*>(st.c[PAR]), c.ste,
                     c.valid, kb, c.qframe, c.lane, ds);
    else
      ds_block<false>(s, dp, c.delta, mk, nullptr, nullptr, false, kb, c.qframe, c.lane, ds);
    tr_mfma<D>(c.dq, ds, ks, c.ktr, kb);
  }
  wait_copies();
  __syncthreads();
}

// With STE (membership STE folded into this pass) the kernel also sums the
// dS of each row's gated keys per class (tile_kv_class >= 0) into LDS slots
// and writes them to ste_partial[h][row][class] for every row it owns.
template <int D, bool STE>
__global__ __launch_bounds__(kThreads, 2) void dq_kernel(HierBwdArgs a, int total) {
  constexpr int CB = STE ? Geo<D>::MBYTES : 16;
  __shared__ __align__(16) char lds_k0[Geo<D>::TILEB], lds_k1[Geo<D>::TILEB];
  __shared__ __align__(16) char lds_v0[Geo<D>::TILEB], lds_v1[Geo<D>::TILEB];
  __shared__ __align__(16) char lds_m0[Geo<D>::MBYTES], lds_m1[Geo<D>::MBYTES];
  __shared__ __align__(16) char lds_c0[CB], lds_c1[CB];
  __shared__ __align__(16) float lds_ste[STE ? kSteClasses * kSteSlots : 4];
  const QStages st = {{lds_k0, lds_k1}, {lds_v0, lds_v1}, {lds_m0, lds_m1}, {lds_c0, lds_c1}};
  const int logical = hier::xcd_logical(blockIdx.x, gridDim.x);
  if (logical >= total) return;
  const int head = logical / a.n_items;
  const int item = logical - head * a.n_items;
  const int32_t* it = a.tile_items + (int64_t)item * 8;

  QCtx<D> c;
  c.a = &a;
  const int tid = threadIdx.x;
  c.lane = tid & 63;
  c.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qbase = it[0], qstride = it[1], qlen = it[2], row_start = it[3], row_count = it[4];
  const int kv_off = it[5], kv_cnt = it[6];
  c.nt = kv_cnt / kSlab;
  // items of <= 32 rows: two waves split the key blocks (dq_tile_split)
  const bool split = row_count <= 32 && c.nt >= 2;
  const int rrel = split ? 0 : c.wave * 32;
  c.active = split ? c.wave < 2 : rrel < row_count;
  c.c2 = a.scale * kLog2e;
  c.gk = reinterpret_cast<const char*>(a.k + (int64_t)head * a.k_sh);
  c.gv = reinterpret_cast<const char*>(a.v + (int64_t)head * a.v_sh);
  c.k_ss_b = (uint32_t)(a.k_ss * 2);
  c.v_ss_b = (uint32_t)(a.v_ss * 2);
  c.kv_idx = a.tile_kv_idx + kv_off;
  c.kv_mask = a.tile_kv_mask + kv_off;
  c.kv_cls = STE ? a.tile_kv_class + kv_off : nullptr;
  c.t1 = STE ? min(max(a.tile_ste_first[item], 0), c.nt) : c.nt;
  // STE slots per wave (a split item's two waves sum into slots of their own,
  // added in a fixed order at the end: the sums do not depend on timing)
  c.ste = lds_ste + (STE ? c.wave * 32 + (c.lane & 31) : 0);
  c.ck.init(c.wave, c.lane);
#pragma unroll
  for (int i = 0; i < Geo<D>::NC; ++i) c.krow[i] = row_read_off<D, kBothRead>(c.lane, i);
#pragma unroll
  for (int db = 0; db < Geo<D>::NDB; ++db) {
    c.ktr[db][0] = tr_read_off<D, kBothRead>(c.lane, db, 0);
    c.ktr[db][1] = tr_read_off<D, kBothRead>(c.lane, db, 1);
  }

  // the lane's query row
  const int r = rrel + (c.lane & 31);
  c.valid = r < row_count;
  const int ri = row_start + (c.valid ? r : 0);
  c.qframe = ri / qlen;
  c.qtok = qbase + c.qframe * qstride + (ri - c.qframe * qlen);
  load_row<D>(c.q, a.q + (int64_t)c.qtok * a.q_ss + (int64_t)head * a.q_sh, c.lane);
  load_row<D>(c.dov, a.dout + (int64_t)c.qtok * a.do_ss + (int64_t)head * a.do_sh, c.lane);
  {
    bf16x8 o[Geo<D>::NC];
    load_row<D>(o, a.o + (int64_t)c.qtok * a.o_ss + (int64_t)head * a.o_sh, c.lane);
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int cc = 0; cc < Geo<D>::NC; ++cc)
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        d0 = fmaf((float)c.dov[cc][e], (float)o[cc][e], d0);
        d1 = fmaf((float)c.dov[cc][e + 1], (float)o[cc][e + 1], d1);
      }
    c.delta = pair_sum(d0 + d1);
  }
  const int64_t srow = (int64_t)head * a.lse_stride_h + c.qtok;
  const float lse = a.lse[srow];
  c.lse2 = lse == -INFINITY ? INFINITY : lse * kLog2e;
  const bool owner = !split || c.wave == 0;   // the wave that writes the row's results
  if (c.valid && c.lane < 32 && owner) {
    a.delta[srow] = -c.delta;
    a.lse2[srow] = c.lse2;
  }
#pragma unroll
  for (int db = 0; db < Geo<D>::NDB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) c.dq[db][i] = 0.f;
  if (STE && c.lane < 32)   // the lane's own slots (its partner lane adds after the first barrier)
#pragma unroll
    for (int cc = 0; cc < kSteClasses; ++cc) c.ste[cc * kSteSlots] = 0.f;

  const int nt = c.nt;
  if (nt > 0) {
    const Idx<D> i0 = load_idx<D>(c.kv_idx, 0, c.ck.idx_off);
    copy_tile<D, kBothRead>(c.gk, c.k_ss_b, c.ck, i0, st.k[0], c.wave);
    copy_tile<D, kBothRead>(c.gv, c.v_ss_b, c.ck, i0, st.v[0], c.wave);
    copy_dwords(c.kv_mask, st.m[0], c.lane);
    if (STE && c.t1 == 0) copy_dwords(c.kv_cls, st.c[0], c.lane);
    Idx<D> inext = load_idx<D>(c.kv_idx, min(1, nt - 1), c.ck.idx_off);
    wait_copies();
    __syncthreads();
    int t = 0;
    if (split) {
      for (; t + 1 < nt; t += 2) {
        dq_tile_split<D, 0, STE>(c, t, inext, st);
        dq_tile_split<D, 1, STE>(c, t + 1, inext, st);
      }
      if (t < nt) dq_tile_split<D, 0, STE>(c, t, inext, st);
      // wave 1's dQ into wave 0's, through the K stage 0 (no copy in flight:
      // the last tile issued none and ended with a barrier)
      float* red = reinterpret_cast<float*>(st.k[0]);
      static_assert(Geo<D>::NDB * 16 * 64 * 4 <= Geo<D>::TILEB, "reduction buffer");
      if (c.wave == 1)
#pragma unroll
        for (int db = 0; db < Geo<D>::NDB; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) red[(db * 16 + i) * 64 + c.lane] = c.dq[db][i];
      __syncthreads();
      if (c.wave == 0)
#pragma unroll
        for (int db = 0; db < Geo<D>::NDB; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) c.dq[db][i] += red[(db * 16 + i) * 64 + c.lane];
    } else if constexpr (!STE) {
      for (; t + 1 < nt; t += 2) {
        dq_tile<D, 0, false>(c, t, inext, st);
        dq_tile<D, 1, false>(c, t + 1, inext, st);
      }
      if (t < nt) dq_tile<D, 0, false>(c, t, inext, st);
    } else {
      // The pipelined tile up to the first tile with a gated key (t1, per
      // item from the class builder; a player row's gated keys, the local-hub
      // keys, end its list), dq_tile_ste from there on.  Two loops rather
      // than a choice per tile: with both variants in one loop body the
      // registers no longer fit.  Tile t sits in stage t & 1.
      const int t1 = c.t1;
      for (; t + 1 < t1; t += 2) {
        dq_tile<D, 0, true>(c, t, inext, st);
        dq_tile<D, 1, true>(c, t + 1, inext, st);
      }
      if (t < t1) dq_tile<D, 0, true>(c, t++, inext, st);
      if (t < nt && (t & 1)) dq_tile_ste<D, 1>(c, t++, inext, st);
      for (; t + 1 < nt; t += 2) {
        dq_tile_ste<D, 0>(c, t, inext, st);
        dq_tile_ste<D, 1>(c, t + 1, inext, st);
      }
      if (t < nt) dq_tile_ste<D, 0>(c, t, inext, st);
    }
  }
  if (c.active && c.valid && owner)
    store_acc<D>(a.dq + (int64_t)c.qtok * a.dq_ss + (int64_t)head * a.dq_sh, c.dq, a.scale, c.lane);
  if constexpr (STE) {
    // every tile ended with a barrier, so both lanes' adds are in the slots
    if (c.valid && c.lane < 32 && owner) {
      float* dst = a.ste_partial + (int64_t)head * a.ste_stride_h + (int64_t)c.qtok * a.ste_classes;
#pragma unroll
      for (int cc = 0; cc < kSteClasses; ++cc)
        if (cc < a.ste_classes)
          dst[cc] = split ? c.ste[cc * kSteSlots] + c.ste[cc * kSteSlots + 32] : c.ste[cc * kSteSlots];
    }
  }
}

// ---- dK, dV (key-major) ------------------------------------------------------

template <int D>
struct KCtx {
  const char* gq;
  const char* gdo;
  const float* lse2;     // head row of the workspace
  const float* delta;
  const int32_t* q_idx;
  const uint32_t* q_mask;
  uint32_t q_ss_b, do_ss_b;
  float c2;
  int nt, wave, lane;
  bool active;
  Copier<D, kBothRead> cq;
  int row[Geo<D>::NC], tr[Geo<D>::NDB][2];
  // the wave's key rows (K^T or V^T operand) and its accumulator (dV^T or dK^T)
  bf16x8 kt[Geo<D>::NC];
  f32x16 acc[Geo<D>::NDB];
  int ktok, kframe;
  bool valid;
};

// ---- dK and dV in one pass: wave pairs share S and P, pipelined over tiles ----
//
// Eight waves per workgroup over one key item of 128 rows; waves w (role A)
// and w+4 (role B) own the same 32 key rows and run on the same SIMD.  Per
// 64-query tile (two 32-query blocks):
//   role A: S = Q K^T, P = exp2(S * c2 - lse2[q]) (0 where the query frame
//           may not see the key frame), P to LDS (fp16), dV^T += dO^T P
//   role B: dP = dO V^T, dS = P * (dP - delta[q]) with P from LDS,
//           dK^T += Q^T dS
// S is computed once for both gradients (four products per block, against
// five for two separate passes).  Step t accumulates tile t (role A: dV from
// the P it kept in registers; role B: dS and dK from the P role A wrote in
// step t-1) while it computes S / P (role A) and dP (role B) of tile t+1, so
// the products of the two roles and of the two tiles overlap on each SIMD;
// one barrier per step hands P over.  Three LDS stages (tiles t, t+1 in use,
// t+2 being copied), two P slots by tile parity; one workgroup per CU.
// P travels as fp16 (10-bit mantissa; P <= 1): dK differs from a P kept in
// fp32 by one rounding of P, dV is unchanged.

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
constexpr int kPairWaves = 8;
constexpr int kPairThreads = 64 * kPairWaves;

template <int D>
__global__ __launch_bounds__(kPairThreads, 1) void dkv_kernel(HierBwdArgs a, int total) {
  __shared__ __align__(16) char lds_q[3][Geo<D>::TILEB];
  __shared__ __align__(16) char lds_d[3][Geo<D>::TILEB];
  __shared__ __align__(16) char lds_w[3][3 * Geo<D>::MBYTES];
  // P of one query tile per wave pair (fp16): [tile parity][block][pair][half][lane]
  __shared__ __align__(16) f16x8 lds_p[2 * 2 * 4 * 2 * 64];
  const int logical = hier::xcd_logical(blockIdx.x, gridDim.x);
  if (logical >= total) return;
  const int head = logical / a.n_key_items;
  const int item = logical - head * a.n_key_items;
  const int32_t* it = a.key_items + (int64_t)item * 8;

  KCtx<D> c;
  const int tid = threadIdx.x;
  c.lane = tid & 63;
  const int wave8 = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool role_b = wave8 >= 4;
  c.wave = wave8 & 3;
  const int kbase = it[0], kstride = it[1], klen = it[2], row_start = it[3], row_count = it[4];
  const int q_off = it[5], q_cnt = it[6];
  c.nt = q_cnt / kSlab;
  // items of <= 32 key rows (a hub stream's keys, a player block's ragged
  // last keys): wave pairs 0 and 1 hold the same rows and take one 32-query
  // block of every tile each (run_split); pairs 2 and 3 only copy
  const bool split = row_count <= 32 && c.nt >= 2;
  const int rrel = split ? 0 : c.wave * 32;
  c.active = split ? c.wave < 2 : rrel < row_count;
  c.c2 = a.scale * kLog2e;
  c.gq = reinterpret_cast<const char*>(a.q + (int64_t)head * a.q_sh);
  c.gdo = reinterpret_cast<const char*>(a.dout + (int64_t)head * a.do_sh);
  c.q_ss_b = (uint32_t)(a.q_ss * 2);
  c.do_ss_b = (uint32_t)(a.do_ss * 2);
  c.lse2 = a.lse2 + (int64_t)head * a.lse_stride_h;
  c.delta = a.delta + (int64_t)head * a.lse_stride_h;
  c.q_idx = a.key_q_idx + q_off;
  c.q_mask = a.key_q_mask + q_off;
  c.cq.init(c.wave, c.lane);
#pragma unroll
  for (int i = 0; i < Geo<D>::NC; ++i) c.row[i] = row_read_off<D, kBothRead>(c.lane, i);
#pragma unroll
  for (int db = 0; db < Geo<D>::NDB; ++db) {
    c.tr[db][0] = tr_read_off<D, kBothRead>(c.lane, db, 0);
    c.tr[db][1] = tr_read_off<D, kBothRead>(c.lane, db, 1);
  }
  const int r = rrel + (c.lane & 31);
  c.valid = r < row_count;
  const int ri = row_start + (c.valid ? r : 0);
  if (kstride < 0) {          // key rows from the row table: (token, key-frame bit) pairs
    c.valid = c.valid && a.key_row_table != nullptr;   // no table: the item has no rows
    const int2 tb =
        c.valid ? reinterpret_cast<const int2*>(a.key_row_table)[kbase + ri] : int2{0, 0};
    c.ktok = tb.x;
    c.kframe = tb.y;
  } else {
    c.kframe = ri / klen;
    c.ktok = kbase + c.kframe * kstride + (ri - c.kframe * klen);
  }
  if (role_b)
    load_row<D>(c.kt, a.v + (int64_t)c.ktok * a.v_ss + (int64_t)head * a.v_sh, c.lane);
  else
    load_row<D>(c.kt, a.k + (int64_t)c.ktok * a.k_ss + (int64_t)head * a.k_sh, c.lane);
#pragma unroll
  for (int db = 0; db < Geo<D>::NDB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) c.acc[db][i] = 0.f;
  f16x8* const pslot = lds_p + c.wave * 2 * 64 + c.lane;   // + par * 1024 + block * 512 + h * 64

  auto copy_q_tile = [&](int t, const Idx<D>& ix, int qtok, int sg) {
    if (role_b) {
      copy_tile<D, kBothRead>(c.gdo, c.do_ss_b, c.cq, ix, lds_d[sg], c.wave);
    } else {
      copy_tile<D, kBothRead>(c.gq, c.q_ss_b, c.cq, ix, lds_q[sg], c.wave);
      if (c.wave == 0) copy_dwords(c.q_mask + t * kSlab, lds_w[sg], c.lane);
      if (c.wave == 1) dma4_lane(c.lse2 + qtok, lds_w[sg] + Geo<D>::MBYTES);
      if (c.wave == 2) dma4_lane(c.delta + qtok, lds_w[sg] + 2 * Geo<D>::MBYTES);
    }
  };
  // role A: S and P of query block qb of tile t (stage sg) into pb (bf16)
  // and the P slot of parity par
  auto a_block = [&](int sg, int par, int qb, bf16x8* pb) {
    const uint32_t* mk = reinterpret_cast<const uint32_t*>(lds_w[sg]);
    const float* l2 = reinterpret_cast<const float*>(lds_w[sg] + Geo<D>::MBYTES);
    f32x16 x = row_mfma<D>(c.kt, lds_q[sg], c.row, qb);
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int q0 = qb * 32 + 8 * g4 + 4 * (c.lane >> 5);
      const u32x4 w = *reinterpret_cast<const u32x4*>(&mk[q0]);
      const u32x4 lw = *reinterpret_cast<const u32x4*>(&l2[q0]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * g4 + e;
        x[i] = __uint_as_float(__float_as_uint(__builtin_amdgcn_exp2f(
                                   fmaf(x[i], c.c2, -__uint_as_float(lw[e])))) &
                               keep_mask(w[e], c.kframe));
        pb[i >> 3][i & 7] = (__bf16)x[i];
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      f16x8 ph;
#pragma unroll
      for (int e = 0; e < 8; ++e) ph[e] = (_Float16)x[8 * h + e];
      pslot[par * 1024 + qb * 512 + h * 64] = ph;
    }
  };
  auto a_front = [&](int sg, int par, bf16x8 (*pb)[2]) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) a_block(sg, par, qb, pb[qb]);
  };
  // role B: dP - delta of query block qb of the tile in stage sg (the
  // products accumulate onto -delta, which the workspace holds per query row)
  auto b_dp = [&](int sg, int qb) {
    const float* dl = reinterpret_cast<const float*>(lds_w[sg] + 2 * Geo<D>::MBYTES);
    f32x16 init;
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const u32x4 dw = *reinterpret_cast<const u32x4*>(&dl[qb * 32 + 8 * g4 + 4 * (c.lane >> 5)]);
#pragma unroll
      for (int e = 0; e < 4; ++e) init[4 * g4 + e] = __uint_as_float(dw[e]);
    }
    return row_mfma_from<D>(init, c.kt, lds_d[sg], c.row, qb);
  };
  // role B: dS = P (dP - delta) of query block qb of tile t from its P slot
  // (one fp16 x fp32 fused multiply per element), then dK^T += Q^T dS
  auto b_block = [&](int sg, int par, int qb, const f32x16& dp) {
    bf16x8 ob[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const f16x8 ph = pslot[par * 1024 + qb * 512 + h * 64];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = 8 * h + e;
        ob[i >> 3][i & 7] = (__bf16)fmaf((float)ph[e], dp[i], 0.f);
      }
    }
    tr_mfma<D>(c.acc, ob, lds_q[sg], c.tr, qb);   // dK^T += Q^T dS
  };
  auto b_back = [&](int sg, int par, const f32x16* dp) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) b_block(sg, par, qb, dp[qb]);
  };

  auto run = [&](auto rb) {
    constexpr bool RB = decltype(rb)::value;
  const int nt = c.nt;
  if (nt > 0) {
    // prologue: tiles 0 and 1 resident; S / P of tile 0 (role A, P slot 0),
    // dP of tile 0 (role B)
    const Idx<D> i0 = load_idx<D>(c.q_idx, 0, c.cq.idx_off);
    copy_q_tile(0, i0, c.q_idx[c.lane], 0);
    if (nt > 1) {
      const Idx<D> i1 = load_idx<D>(c.q_idx, 1, c.cq.idx_off);
      copy_q_tile(1, i1, c.q_idx[kSlab + c.lane], 1);
    }
    const int t2 = min(2, nt - 1);
    Idx<D> inext = load_idx<D>(c.q_idx, t2, c.cq.idx_off);
    int qnext = c.q_idx[t2 * kSlab + c.lane];
    wait_copies();
    __syncthreads();
    bf16x8 pb[2][2];   // role A: P of the current tile (the dV operand)
    f32x16 dp[2];      // role B: dP of the current tile
    if (c.active) {
      if constexpr (!RB) a_front(0, 0, pb);
      else {
        dp[0] = b_dp(0, 0);
        dp[1] = b_dp(0, 1);
      }
    }
    hier::barrier_lds();   // P of tile 0 written
    // iteration t: tiles t (stage s0) and t+1 (s1) resident, P(t) in slot t&1;
    // copies of tile t+2 into s2; role A: S / P of tile t+1 and dV of tile t;
    // role B: dP of tile t+1 and dS / dK of tile t
    int s0 = 0, s1 = 1, s2 = 2;
    // one step; `next` (a constant at both call sites) says whether tile t+1
    // exists, so the steady-state steps carry no branch around the products
    auto step = [&](int t, bool next) {
      if (t + 2 < nt) {
        copy_q_tile(t + 2, inext, qnext, s2);
        const int t3 = min(t + 3, nt - 1);
        inext = load_idx<D>(c.q_idx, t3, c.cq.idx_off);
        qnext = c.q_idx[t3 * kSlab + c.lane];
      }
      if (c.active) {
        if constexpr (!RB) {
          bf16x8 pn[2][2];
          if (next) a_front(s1, (t + 1) & 1, pn);
          tr_mfma<D>(c.acc, pb[0], lds_d[s0], c.tr, 0);   // dV^T += dO^T P
          tr_mfma<D>(c.acc, pb[1], lds_d[s0], c.tr, 1);
          if (next) {
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) { pb[qb][0] = pn[qb][0]; pb[qb][1] = pn[qb][1]; }
          }
        } else {
          f32x16 dn[2];
          if (next) {
            dn[0] = b_dp(s1, 0);
            dn[1] = b_dp(s1, 1);
          }
          b_back(s0, t & 1, dp);
          if (next) { dp[0] = dn[0]; dp[1] = dn[1]; }
        }
      }
      wait_copies();
      __syncthreads();
      const int sx = s0; s0 = s1; s1 = s2; s2 = sx;
    };
    int t = 0;
    for (; t + 1 < nt; ++t) step(t, true);
    step(t, false);
  }
  };
  // the same schedule for a split item: pair w takes query block w of every
  // tile (its own P slot), one block of products per tile and role
  auto run_split = [&](auto rb) {
    constexpr bool RB = decltype(rb)::value;
    const int nt = c.nt;
    const int qb = c.wave;
    const Idx<D> i0 = load_idx<D>(c.q_idx, 0, c.cq.idx_off);
    copy_q_tile(0, i0, c.q_idx[c.lane], 0);
    const Idx<D> i1 = load_idx<D>(c.q_idx, 1, c.cq.idx_off);   // nt >= 2
    copy_q_tile(1, i1, c.q_idx[kSlab + c.lane], 1);
    const int t2 = min(2, nt - 1);
    Idx<D> inext = load_idx<D>(c.q_idx, t2, c.cq.idx_off);
    int qnext = c.q_idx[t2 * kSlab + c.lane];
    wait_copies();
    __syncthreads();
    bf16x8 pb[2];   // role A: P of block qb of the current tile
    f32x16 dp;      // role B: dP of block qb of the current tile
    if (c.active) {
      if constexpr (!RB) a_block(0, 0, qb, pb);
      else dp = b_dp(0, qb);
    }
    hier::barrier_lds();   // P of tile 0 written
    int s0 = 0, s1 = 1, s2 = 2;
    auto step = [&](int t, bool next) {
      if (t + 2 < nt) {
        copy_q_tile(t + 2, inext, qnext, s2);
        const int t3 = min(t + 3, nt - 1);
        inext = load_idx<D>(c.q_idx, t3, c.cq.idx_off);
        qnext = c.q_idx[t3 * kSlab + c.lane];
      }
      if (c.active) {
        if constexpr (!RB) {
          bf16x8 pn[2];
          if (next) a_block(s1, (t + 1) & 1, qb, pn);
          tr_mfma<D>(c.acc, pb, lds_d[s0], c.tr, qb);   // dV^T += dO^T P
          if (next) { pb[0] = pn[0]; pb[1] = pn[1]; }
        } else {
          f32x16 dn;
          if (next) dn = b_dp(s1, qb);
          b_block(s0, t & 1, qb, dp);
          if (next) dp = dn;
        }
      }
      wait_copies();
      __syncthreads();
      const int sx = s0; s0 = s1; s1 = s2; s2 = sx;
    };
    int t = 0;
    for (; t + 1 < nt; ++t) step(t, true);
    step(t, false);
    // pair 1's sums into pair 0's, through the Q stages (no copy in flight:
    // the last steps issued none and ended with a barrier)
    float* red = reinterpret_cast<float*>(lds_q[RB ? 1 : 0]);
    static_assert(Geo<D>::NDB * 16 * 64 * 4 <= Geo<D>::TILEB, "reduction buffer");
    if (c.wave == 1)
#pragma unroll
      for (int db = 0; db < Geo<D>::NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) red[(db * 16 + i) * 64 + c.lane] = c.acc[db][i];
    __syncthreads();
    if (c.wave == 0)
#pragma unroll
      for (int db = 0; db < Geo<D>::NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) c.acc[db][i] += red[(db * 16 + i) * 64 + c.lane];
  };
  if (split) {
    if (role_b) run_split(std::true_type{});
    else run_split(std::false_type{});
  } else {
    if (role_b) run(std::true_type{});
    else run(std::false_type{});
  }
  if (c.active && c.valid && (!split || c.wave == 0)) {
    if (role_b)
      store_acc<D>(a.dk + (int64_t)c.ktok * a.dk_ss + (int64_t)head * a.dk_sh, c.acc, a.scale, c.lane);
    else
      store_acc<D>(a.dv + (int64_t)c.ktok * a.dv_ss + (int64_t)head * a.dv_sh, c.acc, 1.f, c.lane);
  }
}

// ---- membership STE partial sums (query-major, gated keys only) -------------

// LDS: K[2] | V[2] (rows) | masks[2] | classes[2] | per-wave row sums
template <int D>
struct SLds {
  static constexpr int KOFF = 0;
  static constexpr int VOFF = 2 * Geo<D>::TILEB;
  static constexpr int MOFF = 4 * Geo<D>::TILEB;
  static constexpr int COFF = MOFF + 2 * Geo<D>::MBYTES;
  static constexpr int AOFF = COFF + 2 * Geo<D>::MBYTES;
  static constexpr int SIZE = AOFF + kSteClasses * kWaves * 32 * 4;
};

template <int D>
__global__ __launch_bounds__(kThreads, 2) void ste_kernel(HierBwdArgs a, int total) {
  __shared__ __align__(16) char lds[SLds<D>::SIZE];
  const int logical = hier::xcd_logical(blockIdx.x, gridDim.x);
  if (logical >= total) return;
  const int head = logical / a.n_ste_items;
  const int item = logical - head * a.n_ste_items;
  const int32_t* it = a.ste_items + (int64_t)item * 8;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qbase = it[0], qstride = it[1], qlen = it[2], row_start = it[3], row_count = it[4];
  const int kv_off = it[5], kv_cnt = it[6];
  const int nt = kv_cnt / kSlab;
  const bool active = wave * 32 < row_count;
  const float c2 = a.scale * kLog2e;
  const char* gk = reinterpret_cast<const char*>(a.k + (int64_t)head * a.k_sh);
  const char* gv = reinterpret_cast<const char*>(a.v + (int64_t)head * a.v_sh);
  const uint32_t k_ss_b = (uint32_t)(a.k_ss * 2), v_ss_b = (uint32_t)(a.v_ss * 2);
  const int32_t* kv_idx = a.ste_kv_idx + kv_off;
  const uint32_t* kv_mask = a.ste_kv_mask + kv_off;
  const int32_t* kv_cls = a.ste_kv_class + kv_off;
  Copier<D, kRowRead> cp;
  cp.init(wave, lane);
  int roff[Geo<D>::NC];
#pragma unroll
  for (int i = 0; i < Geo<D>::NC; ++i) roff[i] = row_read_off<D, kRowRead>(lane, i);

  // Per-query partial sums, one slot per (class, query row of the workgroup):
  // acc[class * 128 + wave * 32 + (lane & 31)].  Only the two lanes of a query
  // (its two key halves) share a slot, whatever the classes of the keys, so an
  // add conflicts at most two ways.
  constexpr int kSlots = kWaves * 32;
  float* acc = reinterpret_cast<float*>(lds + SLds<D>::AOFF) + wave * 32 + (lane & 31);
  if (lane < 32)
#pragma unroll
    for (int cc = 0; cc < kSteClasses; ++cc) acc[cc * kSlots] = 0.f;

  if (row_count <= 32) {
    // At most 32 rows (a hub slot's rows against long key lists): the four
    // waves share the rows and split the 32-key blocks (wave w takes blocks w,
    // w + 4, ...), reading K and V rows straight into the MFMA operand
    // registers, so the loop has no LDS stages and no barriers.  Each wave
    // sums into its own slots; the four are added in wave order at the end.
    const int r = lane & 31;
    const bool valid = r < row_count;
    const int ri = row_start + (valid ? r : 0);
    const int qframe = ri / qlen;
    const int qtok = qbase + qframe * qstride + (ri - qframe * qlen);
    bf16x8 q[Geo<D>::NC], dov[Geo<D>::NC];
    load_row<D>(q, a.q + (int64_t)qtok * a.q_ss + (int64_t)head * a.q_sh, lane);
    load_row<D>(dov, a.dout + (int64_t)qtok * a.do_ss + (int64_t)head * a.do_sh, lane);
    const int64_t srow = (int64_t)head * a.lse_stride_h + qtok;
    const float lse2 = a.lse2[srow], delta = -a.delta[srow];
    const int nb = kv_cnt / 32;
    for (int j = wave; j < nb; j += kWaves) {
      const int64_t key = kv_idx[32 * j + r];
      // operand layout of row_mfma: lane l holds elements 16c + 8(l/32) .. +8
      // of key row 32j + l%32 in its k-step c
      const char* kp = gk + key * k_ss_b + 16 * (lane >> 5);
      const char* vp = gv + key * v_ss_b + 16 * (lane >> 5);
      bf16x8 ka[Geo<D>::NC], va[Geo<D>::NC];
#pragma unroll
      for (int c = 0; c < Geo<D>::NC; ++c) {
        ka[c] = *reinterpret_cast<const bf16x8*>(kp + 32 * c);
        va[c] = *reinterpret_cast<const bf16x8*>(vp + 32 * c);
      }
      const f32x16 zero = {};
      f32x16 s = mfma(ka[0], q[0], zero), dp = mfma(va[0], dov[0], zero);
#pragma unroll
      for (int c = 1; c < Geo<D>::NC; ++c) {
        s = mfma(ka[c], q[c], s);
        dp = mfma(va[c], dov[c], dp);
      }
      float ds[16];
      uint32_t cls[16];
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int k0 = 32 * j + 8 * g4 + 4 * (lane >> 5);
        const u32x4 w = *reinterpret_cast<const u32x4*>(&kv_mask[k0]);
        const u32x4 cl = *reinterpret_cast<const u32x4*>(&kv_cls[k0]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * g4 + e;
          const float p = __builtin_amdgcn_exp2f(fmaf(s[i], c2, -lse2));
          ds[i] = __uint_as_float(__float_as_uint(p * (dp[i] - delta)) & keep_mask(w[e], qframe));
          cls[i] = cl[e];   // >= kSteClasses (or -1): dropped by ste_add
        }
      }
      ste_add(acc, ds, cls, valid);
    }
    __syncthreads();
    if (wave == 0 && valid && lane < 32) {
      const float* sum = reinterpret_cast<const float*>(lds + SLds<D>::AOFF) + lane;
      float* dst = a.ste_partial + (int64_t)head * a.ste_stride_h + (int64_t)qtok * a.ste_classes;
#pragma unroll
      for (int cc = 0; cc < kSteClasses; ++cc)
        if (cc < a.ste_classes) {
          float t = sum[cc * kSlots];
#pragma unroll
          for (int w = 1; w < kWaves; ++w) t += sum[cc * kSlots + 32 * w];
          dst[cc] = t;
        }
    }
    return;
  }

  const int r = wave * 32 + (lane & 31);
  const bool valid = r < row_count;
  const int ri = row_start + (valid ? r : 0);
  const int qframe = ri / qlen;
  const int qtok = qbase + qframe * qstride + (ri - qframe * qlen);
  bf16x8 q[Geo<D>::NC], dov[Geo<D>::NC];
  load_row<D>(q, a.q + (int64_t)qtok * a.q_ss + (int64_t)head * a.q_sh, lane);
  load_row<D>(dov, a.dout + (int64_t)qtok * a.do_ss + (int64_t)head * a.do_sh, lane);
  const int64_t srow = (int64_t)head * a.lse_stride_h + qtok;
  const float lse2 = a.lse2[srow], delta = -a.delta[srow];

  // Tile t+1 is copied into the other stage while tile t is processed.
  auto copy = [&](int t, const Idx<D>& ix) {
    const int par = t & 1;
    copy_tile<D, kRowRead>(gk, k_ss_b, cp, ix, lds + SLds<D>::KOFF + par * Geo<D>::TILEB, wave);
    copy_tile<D, kRowRead>(gv, v_ss_b, cp, ix, lds + SLds<D>::VOFF + par * Geo<D>::TILEB, wave);
    copy_dwords(kv_mask + t * kSlab, lds + SLds<D>::MOFF + par * Geo<D>::MBYTES, lane);
    copy_dwords(kv_cls + t * kSlab, lds + SLds<D>::COFF + par * Geo<D>::MBYTES, lane);
  };
  if (nt > 0) copy(0, load_idx<D>(kv_idx, 0, cp.idx_off));
  Idx<D> inext = load_idx<D>(kv_idx, min(1, max(nt - 1, 0)), cp.idx_off);
  wait_copies();
  __syncthreads();
  for (int t = 0; t < nt; ++t) {
    const int par = t & 1;
    if (t + 1 < nt) copy(t + 1, inext);
    inext = load_idx<D>(kv_idx, min(t + 2, nt - 1), cp.idx_off);
    const char* ks = lds + SLds<D>::KOFF + par * Geo<D>::TILEB;
    const char* vs = lds + SLds<D>::VOFF + par * Geo<D>::TILEB;
    const uint32_t* mk = reinterpret_cast<const uint32_t*>(lds + SLds<D>::MOFF + par * Geo<D>::MBYTES);
    const int32_t* ck = reinterpret_cast<const int32_t*>(lds + SLds<D>::COFF + par * Geo<D>::MBYTES);
    if (active) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const f32x16 s = row_mfma<D>(q, ks, roff, kb);
        const f32x16 dp = row_mfma<D>(dov, vs, roff, kb);
        float ds[16];
        uint32_t cls[16];
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int k0 = kb * 32 + 8 * g4 + 4 * (lane >> 5);
          const u32x4 w = *reinterpret_cast<const u32x4*>(&mk[k0]);
          const u32x4 cl = *reinterpret_cast<const u32x4*>(&ck[k0]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = 4 * g4 + e;
            const float p = __builtin_amdgcn_exp2f(fmaf(s[i], c2, -lse2));
            ds[i] = __uint_as_float(__float_as_uint(p * (dp[i] - delta)) & keep_mask(w[e], qframe));
            cls[i] = cl[e];   // >= kSteClasses (or -1): dropped by ste_add
          }
        }
        ste_add(acc, ds, cls, valid);
      }
    }
    wait_copies();
    __syncthreads();
  }
  if (active && valid && lane < 32) {
    float* dst = a.ste_partial + (int64_t)head * a.ste_stride_h + (int64_t)qtok * a.ste_classes;
#pragma unroll
    for (int cc = 0; cc < kSteClasses; ++cc)
      if (cc < a.ste_classes) dst[cc] = acc[cc * kSlots];
  }
}


// Argument checks and the launches of both entry points (a is complete: the
// workspace pointers are set).
int bwd_run(const HierBwdArgs& a, void* stream) {
  HIER_REQUIRE(a.D == 128 || a.D == 64, HIER_EUNSUPPORTED, "head_dim must be 64 or 128, got %d", a.D);
  HIER_REQUIRE(a.H >= 1 && a.n_items >= 0 && a.n_key_items >= 0 && a.kv_rows >= 0 && a.q_rows >= 0,
               HIER_EINVAL, "invalid H=%d n_items=%d n_key_items=%d", a.H, a.n_items, a.n_key_items);
  HIER_REQUIRE(a.q && a.k && a.v && a.o && a.dout && a.lse && a.delta && a.lse2 && a.dq && a.dk &&
                   a.dv && a.tile_items && a.tile_kv_idx && a.tile_kv_mask && a.tile_blk_and &&
                   a.key_items && a.key_q_idx && a.key_q_mask && a.key_blk_and,
               HIER_EINVAL, "NULL pointer");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  HIER_REQUIRE(al16(a.q) && al16(a.k) && al16(a.v) && al16(a.o) && al16(a.dout) && al16(a.dq) &&
                   al16(a.dk) && al16(a.dv) && al16(a.tile_kv_idx) && al16(a.key_q_idx),
               HIER_EINVAL, "tensors and index lists must be 16-byte aligned");
  const int64_t st[] = {a.q_ss, a.q_sh, a.k_ss, a.k_sh, a.v_ss, a.v_sh, a.o_ss, a.o_sh,
                        a.do_ss, a.do_sh, a.dq_ss, a.dq_sh, a.dk_ss, a.dk_sh, a.dv_ss, a.dv_sh};
  for (int64_t s : st)
    HIER_REQUIRE(s >= 0 && s % 8 == 0, HIER_EINVAL, "strides must be non-negative multiples of 8");
  constexpr __int128 k4G = (__int128)1 << 32;
  HIER_REQUIRE(hier::span_bytes(a.kv_rows, a.k_ss, a.k_sh, a.H, a.D) <= k4G &&
                   hier::span_bytes(a.kv_rows, a.v_ss, a.v_sh, a.H, a.D) <= k4G &&
                   hier::span_bytes(a.q_rows, a.q_ss, a.q_sh, a.H, a.D) <= k4G &&
                   hier::span_bytes(a.q_rows, a.do_ss, a.do_sh, a.H, a.D) <= k4G,
               HIER_EUNSUPPORTED, "Q/K/V/dO views must span at most 4 GiB");
  HIER_REQUIRE(copy_rows_ok(a.kv_rows, a.k_ss) && copy_rows_ok(a.kv_rows, a.v_ss) &&
                   copy_rows_ok(a.q_rows, a.q_ss) && copy_rows_ok(a.q_rows, a.do_ss),
               HIER_EUNSUPPORTED,
               "Q/K/V/dO need at most 2^24 rows and a row stride under 8M elements");
  HIER_REQUIRE(a.n_ste_items >= 0, HIER_EINVAL, "n_ste_items must be >= 0");
  if (a.n_ste_items > 0) {
    HIER_REQUIRE(a.ste_items && a.ste_kv_idx && a.ste_kv_mask && a.ste_kv_class && a.ste_partial &&
                     al16(a.ste_kv_idx) && al16(a.ste_kv_mask) && al16(a.ste_kv_class),
                 HIER_EINVAL, "membership STE: NULL or misaligned list");
    HIER_REQUIRE(a.ste_classes >= 1 && a.ste_classes <= kSteClasses, HIER_EUNSUPPORTED,
                 "membership STE supports 1..%d classes (groups / players), got %d", kSteClasses,
                 a.ste_classes);
    HIER_REQUIRE((int64_t)a.n_ste_items * a.H <= hier::kMaxLaunchItems, HIER_EUNSUPPORTED,
                 "too many work items");
  }
  const bool fold = a.tile_kv_class != nullptr;
  if (fold) {
    HIER_REQUIRE(a.n_ste_items == 0, HIER_EINVAL,
                 "membership STE: tile_kv_class (in the dQ pass) and an STE list are exclusive");
    HIER_REQUIRE(a.ste_partial && a.tile_ste_first && al16(a.tile_kv_class), HIER_EINVAL,
                 "membership STE: NULL ste_partial / tile_ste_first or misaligned tile_kv_class");
    HIER_REQUIRE(a.ste_classes >= 1 && a.ste_classes <= kSteClasses, HIER_EUNSUPPORTED,
                 "membership STE supports 1..%d classes (groups / players), got %d", kSteClasses,
                 a.ste_classes);
  }
  const int64_t tq = (int64_t)a.n_items * a.H, tk = (int64_t)a.n_key_items * a.H;
  HIER_REQUIRE(tq <= hier::kMaxLaunchItems && tk <= hier::kMaxLaunchItems, HIER_EUNSUPPORTED, "too many work items");
  hipStream_t s = (hipStream_t)stream;
  if (tq > 0) {
    const int grid = (int)hier::xcd_grid(tq);
    if (a.D == 128 && fold)
      hipLaunchKernelGGL((dq_kernel<128, true>), dim3(grid), dim3(kThreads), 0, s, a, (int)tq);
    else if (a.D == 128)
      hipLaunchKernelGGL((dq_kernel<128, false>), dim3(grid), dim3(kThreads), 0, s, a, (int)tq);
    else if (fold)
      hipLaunchKernelGGL((dq_kernel<64, true>), dim3(grid), dim3(kThreads), 0, s, a, (int)tq);
    else
      hipLaunchKernelGGL((dq_kernel<64, false>), dim3(grid), dim3(kThreads), 0, s, a, (int)tq);
    int rc = hier::check_launch("dq_kernel");
    if (rc != HIER_OK) return rc;
  }
  if (tk > 0) {
    const int grid = (int)hier::xcd_grid(tk);
    if (a.D == 128)
      hipLaunchKernelGGL(dkv_kernel<128>, dim3(grid), dim3(kPairThreads), 0, s, a, (int)tk);
    else
      hipLaunchKernelGGL(dkv_kernel<64>, dim3(grid), dim3(kPairThreads), 0, s, a, (int)tk);
    int rc = hier::check_launch("dkv_kernel");
    if (rc != HIER_OK) return rc;
  }
  const int64_t ts = (int64_t)a.n_ste_items * a.H;
  if (a.n_ste_items > 0) {
    const int grid = (int)hier::xcd_grid(ts);
    if (a.D == 128)
      hipLaunchKernelGGL(ste_kernel<128>, dim3(grid), dim3(kThreads), 0, s, a, (int)ts);
    else
      hipLaunchKernelGGL(ste_kernel<64>, dim3(grid), dim3(kThreads), 0, s, a, (int)ts);
    return hier::check_launch("ste_kernel");
  }
  return HIER_OK;
}

// ---- workspace of the allocation-free entry point ---------------------------

// delta and lse2 of hier_attn_bwd_noalloc: [H][lse_stride_h] floats each, in
// this file-scope device array.  Each GPU the library runs on holds its own
// copy until the process ends; every call on that GPU uses it, so calls that
// overlap on one GPU (two streams, two threads) race.
constexpr int64_t kScratchFloats = 4ll << 20;   // 16 MiB
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device.  The host-side symbol is
// only a stand-in; the address comes from hipGetSymbolAddress, once per
// device, with that device current.
int scratch_ptr(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hier::fail(HIER_ELAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  HIER_REQUIRE(dev >= 0 && dev < kMaxDevices, HIER_EUNSUPPORTED, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return hier::fail(HIER_ELAUNCH, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return HIER_OK;
}

// Zero n floats (n % 4 == 0) with vector stores.  A kernel rather than
// hipMemsetAsync so that the call stays correct inside captured graphs.
__global__ void zero_kernel(float* p, int64_t n4) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  float4* q = reinterpret_cast<float4*>(p);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride)
    q[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

}  // namespace

extern "C" int hier_attn_bwd(const HierBwdArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  return bwd_run(*args, stream);
}

extern "C" int hier_attn_bwd_noalloc(const HierBwdArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  HIER_REQUIRE(args->delta == nullptr && args->lse2 == nullptr, HIER_EINVAL,
               "hier_attn_bwd_noalloc uses the library's device workspace: delta and lse2 must "
               "be NULL");
  HIER_REQUIRE(args->H >= 1 && args->lse_stride_h >= 0, HIER_EINVAL,
               "invalid H=%d lse_stride_h=%lld", args->H, (long long)args->lse_stride_h);
  HIER_REQUIRE(args->H <= kScratchFloats && args->lse_stride_h <= kScratchFloats,
               HIER_EUNSUPPORTED,
               "hier_attn_bwd_noalloc workspace holds 2 x H x lse_stride_h <= %lld floats; got "
               "H=%d x lse_stride_h=%lld",
               (long long)kScratchFloats, args->H, (long long)args->lse_stride_h);
  // delta and lse2 each take H rows of lse_stride_h floats, rounded to 64
  // floats so that lse2 starts 256-byte aligned
  const int64_t per = ((int64_t)args->H * args->lse_stride_h + 63) / 64 * 64;
  HIER_REQUIRE(2 * per <= kScratchFloats, HIER_EUNSUPPORTED,
               "hier_attn_bwd_noalloc workspace holds 2 x H x lse_stride_h <= %lld floats (%lld "
               "MiB); got H=%d x lse_stride_h=%lld",
               (long long)kScratchFloats, (long long)(kScratchFloats * 4 >> 20), args->H,
               (long long)args->lse_stride_h);
  float* ws = nullptr;
  int rc = scratch_ptr(&ws);
  if (rc != HIER_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  // rows no item writes are read as 0, as from a zero-filled caller workspace
  const int64_t n4 = 2 * per / 4;
  if (n4 > 0) {
    const int blocks = (int)std::min<int64_t>((n4 + 255) / 256, 2048);
    hipLaunchKernelGGL(zero_kernel, dim3(blocks), dim3(256), 0, s, ws, n4);
    rc = hier::check_launch("zero_kernel");
    if (rc != HIER_OK) return rc;
  }
  HierBwdArgs a = *args;
  a.delta = ws;
  a.lse2 = ws + per;
  return bwd_run(a, stream);
}

// ---- membership-STE sums reduced to [T, N, P] ------------------------------
//
// out[t][g][p] = sum over heads and the L rows of player p at frame t of
// partial[h][row][g]  +  sum over heads and the KL rows of local hub g at
// frame t of partial[h][row][p]   (full-sequence token order).  One
// workgroup per output; each thread sums a fixed strided subset, then a
// fixed-order tree in LDS: deterministic.
namespace {

__global__ __launch_bounds__(256) void ste_reduce_kernel(HierSteReduceArgs a) {
  __shared__ float part[256];
  const int o = blockIdx.x;
  const int p = o % a.P, g = (o / a.P) % a.N, t = o / (a.P * a.N);
  const int64_t a0 = (int64_t)a.P * a.T * a.L;
  // a head's terms are its L player rows (class g) then its KL hub rows
  // (class p); thread j sums term j, j + 256, ... of every head, head by head
  // (no divisions in the loop, consecutive threads on consecutive rows)
  const int64_t pl0 = ((int64_t)p * a.T + t) * a.L;              // player p's rows at frame t
  const int64_t hub0 = a0 + ((int64_t)t * a.N + g) * a.KL;        // group g's hub rows at frame t
  float s = 0.f;
  for (int j = threadIdx.x; j < a.L + a.KL; j += blockDim.x) {
    const int64_t off = j < a.L ? (pl0 + j) * a.classes + g : (hub0 + j - a.L) * a.classes + p;
#pragma unroll 8
    for (int h = 0; h < a.H; ++h) s += a.partial[(int64_t)h * a.stride_h + off];
  }
  part[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if (threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) a.out[o] = part[0];
}

}  // namespace

extern "C" int hier_ste_reduce(const HierSteReduceArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  const HierSteReduceArgs& a = *args;
  HIER_REQUIRE(a.H >= 1 && a.P >= 1 && a.T >= 1 && a.L >= 1 && a.N >= 1 && a.KL >= 0 &&
                   a.H <= (1 << 16) && a.P <= (1 << 16) && a.T <= (1 << 16) && a.L <= (1 << 20) &&
                   a.N <= (1 << 16) && a.KL <= (1 << 20),
               HIER_EINVAL, "invalid H=%d P=%d T=%d L=%d N=%d KL=%d", a.H, a.P, a.T, a.L, a.N,
               a.KL);
  HIER_REQUIRE(a.classes >= a.P && a.classes >= a.N && a.classes <= kSteClasses, HIER_EINVAL,
               "classes must cover P and N and be at most %d, got %d", kSteClasses, a.classes);
  const int64_t rows = (int64_t)a.P * a.T * a.L + (int64_t)a.T * a.N * a.KL;
  HIER_REQUIRE(a.stride_h >= rows * a.classes, HIER_EINVAL,
               "stride_h %lld below rows x classes %lld", (long long)a.stride_h,
               (long long)(rows * a.classes));
  HIER_REQUIRE((int64_t)a.H * a.L <= INT32_MAX / 2 && (int64_t)a.H * a.KL <= INT32_MAX / 2,
               HIER_EUNSUPPORTED, "too many terms per sum");
  HIER_REQUIRE(a.partial && a.out, HIER_EINVAL, "NULL pointer");
  const int64_t n_out = (int64_t)a.T * a.N * a.P;
  HIER_REQUIRE(n_out <= INT32_MAX, HIER_EUNSUPPORTED, "too many outputs");
  hipLaunchKernelGGL(ste_reduce_kernel, dim3((unsigned)n_out), dim3(256), 0, (hipStream_t)stream,
                     a);
  return hier::check_launch("ste_reduce_kernel");
}
