// Block-sparse, frame-causal flash-attention forward for gfx950 (CDNA4).
//
// Work item = up to 128 query rows of one stream (a player, a local-hub slot or
// the global hub) of one temporal block, for one head.  The rows attend to the
// stream's key list (the ordered union over the block's query frames of the
// reference's per-frame key lists, hier_segmented_attention.py:276-368) with a
// per-key bitmask saying which query frames may see it.  Only listed keys are
// visited; there is no dense S x S mask anywhere.
//
// Math (v_mfma_f32_32x32x16_bf16), per 32-row sub-block and 32-key block:
//   S^T[key, q]  = K[key, :] . Q[q, :]            D/16 MFMAs
//   online softmax over keys: each lane owns one query and 16 keys per block;
//   max / sum are in-register plus one swap with lane^32 (v_permlane32_swap)
//   O^T[d, q]   += V^T[d, key] . P^T[key, q]       D/32 x 2 MFMAs
// The P^T operand comes straight from the S^T registers; the matching V^T
// operand is read with ds_read_b64_tr_b16 (each 16-lane group reads a 4 x 16
// block and lane i receives column i), two reads per MFMA.  fp32 m / l / O, P
// rounded to bf16 before P.V, exp2 with the log2(e)-scaled softmax scale folded
// into one FMA -- the numerics of the reference kernels
// (hier_tiled_attention.py:112-143); the row sum l adds the bf16-rounded P
// (v_dot2_f32_bf16), i.e. exactly the weights that multiply V.  The running max
// is refreshed lazily: a block's P is computed against the running max of the
// blocks before it, so the exps need no block max first; only when a lane's
// block sum exceeds 16 * 2^8 (some score more than 2^8 above that max in exp2
// units; always at a row's first visible key) does the wave take the block
// max, recompute P and rescale O and l.  An accepted P is thus at most 2^12.
// Rows with no visible key output 0
// (hier_segmented_attention.py:104-109).
//
// Workgroup = 4 waves x 32 query rows (128 rows per work item), two
// workgroups per CU.  Keys stream through LDS in 64-key tiles that the waves
// copy with global_load_lds_dwordx4 (HBM/L2 -> LDS, no VGPR staging).  Each
// wave runs a three-stage software pipeline over 32-key blocks whose stages
// are independent within one step, so the softmax VALU work overlaps both
// matrix products:
//     step j:  QK(j+2)  ||  softmax(j+1)  ||  PV(j)
// While the two blocks of tile t are multiplied by V, K tile t+2 (with its
// masks) and V tile t+1 are in flight; two K, two V and two mask stages fill
// 65 KB of LDS per workgroup.
//
// The LDS tile layout and the copies are described in hier_tile.h.
#include "hier_common.h"
#include "hier_launch.h"
#include "hier_tile.h"

namespace {

using namespace hier::tile;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
// A lane's sum of its 16 P values of a block (each 2^(score - running max) in
// exp2 units) above this bound refreshes the running max.
constexpr float kSumMax = 16.f * 256.f;
// Running max of a row that has seen no visible key: finite, so the exp2
// offset -m * c2 stays finite, and a masked score (-inf) still gives P = 0.
constexpr float kNoMax = -1e30f;
constexpr int kValuPerMfma = 3;       // softmax VALU instructions scheduled after each MFMA
constexpr bool kSplitSmall = true;     // items of <= 32 rows: two waves split the key blocks

// LDS stages of a workgroup: K[2], V[2], masks[2] (one dword per key), each
// its own __shared__ array.  K tiles are only read as rows, V tiles only
// transposed.  Distinct arrays let the compiler see that the copies into one
// stage never alias the reads of the other; given one array it waits for every
// outstanding copy before the first LDS read that follows them.
struct Stages {
  char* k[2];
  char* v[2];
  char* m[2];
};

// ---- per-sub-block state and math ------------------------------------------

template <int D>
struct Rows {
  bf16x8 q[Geo<D>::NC];
  f32x16 o[Geo<D>::NDB];
  float m, l, alpha;
  int qtok, qframe;
  bool valid;
  uint32_t bits;   // OR over the sub-block's valid rows of 1 << query frame
};

template <int D>
__device__ __forceinline__ void rows_init(Rows<D>& R, const HierFwdArgs& a, const int32_t* it,
                                          int head, int rrel, int lane) {
  const int qbase = it[0], qstride = it[1], qlen = it[2], row_start = it[3], row_count = it[4];
  const int r = rrel + (lane & 31);
  R.valid = r < row_count;
  const int ri = row_start + (R.valid ? r : 0);
  if (qstride < 0) {            // rows from the row table: (token, mask bit) pairs
    R.valid = R.valid && a.row_table != nullptr;   // no table: the item has no rows
    const int2 tb = R.valid ? reinterpret_cast<const int2*>(a.row_table)[qbase + ri] : int2{0, 0};
    R.qtok = tb.x;
    R.qframe = tb.y;
  } else {
    R.qframe = ri / qlen;
    R.qtok = qbase + R.qframe * qstride + (ri - R.qframe * qlen);
  }
  R.bits = wave_or(R.valid ? (1u << R.qframe) : 0u);
  const uint16_t* qp = a.q + (int64_t)R.qtok * a.q_ss + (int64_t)head * a.q_sh + 8 * (lane >> 5);
#pragma unroll
  for (int c = 0; c < Geo<D>::NC; ++c) R.q[c] = *reinterpret_cast<const bf16x8*>(qp + 16 * c);
#pragma unroll
  for (int db = 0; db < Geo<D>::NDB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) R.o[db][i] = 0.f;
  R.m = kNoMax;
  R.l = 0.f;
  R.alpha = 1.f;
}

// Per-lane LDS byte offsets of the MFMA operand reads (tile-relative).
template <int D>
struct ReadAddr {
  int k[Geo<D>::NC];     // K rows: key (lane & 31), chunk (lane >> 5) + 2c
  int v[Geo<D>::NDB];    // first transposed V read of d-block db, key chunk 0
  __device__ __forceinline__ void init(int lane) {
#pragma unroll
    for (int c = 0; c < Geo<D>::NC; ++c) k[c] = row_read_off<D, kRowRead>(lane, c);
#pragma unroll
    for (int db = 0; db < Geo<D>::NDB; ++db) v[db] = tr_read_off<D, kTrRead>(lane, db, 0);
  }
};

// S^T of 32-key block kb of a tile.
template <int D>
__device__ __forceinline__ f32x16 qk_block(const bf16x8* q, const char* kslot, const ReadAddr<D>& ra,
                                           int kb) {
  const char* base = kslot + kb * 32 * Geo<D>::ROWB;
  const f32x16 zero = {};
  f32x16 s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
      *reinterpret_cast<const bf16x8*>(base + ra.k[0]), q[0], zero, 0, 0, 0);
#pragma unroll
  for (int c = 1; c < Geo<D>::NC; ++c)
    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*reinterpret_cast<const bf16x8*>(base + ra.k[c]),
                                                q[c], s, 0, 0, 0);
  return s;
}

// Set the scores of block kb that the lane's query frame may not see to -inf.
__device__ __forceinline__ void mask_block(f32x16& s, const char* mslot, int kb, int qframe,
                                           int lane) {
  const uint32_t* mk = reinterpret_cast<const uint32_t*>(mslot);
#pragma unroll
  for (int g4 = 0; g4 < 4; ++g4) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(&mk[kb * 32 + 8 * g4 + 4 * (lane >> 5)]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t sel = (uint32_t)__builtin_amdgcn_sbfe((int)w[e], qframe, 1);
      const uint32_t x = __float_as_uint(s[4 * g4 + e]);
      s[4 * g4 + e] = __uint_as_float((x & sel) | (0xff800000u & ~sel));
    }
  }
}

// P of one 32-key block: exp2(s * c2 + nb) rounded to bf16, written as the
// two P^T operands of the block; returns the lane's sum of the rounded P
// (v_dot2_f32_bf16 against ones), i.e. exactly the weights that multiply V.
__device__ __forceinline__ float p_block(const f32x16& s, bf16x8* p, float c2, float nb) {
#pragma unroll
  for (int i = 0; i < 16; ++i)
    p[i >> 3][i & 7] = (__bf16)__builtin_amdgcn_exp2f(fmaf(s[i], c2, nb));
  const bf16x2 one = {(__bf16)1.f, (__bf16)1.f};
  float ps0 = 0.f, ps1 = 0.f;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    ps0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p[c], p[c], 0, 1), one, ps0, false);
    ps1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p[c], p[c], 2, 3), one, ps1, false);
    ps0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p[c], p[c], 4, 5), one, ps0, false);
    ps1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p[c], p[c], 6, 7), one, ps1, false);
  }
  return ps0 + ps1;
}

// Online softmax, second half: ps is the lane's sum of a block's P taken
// against the running max R.m (p_block with nb = -R.m * c2).  While every
// lane's sum stays <= kSumMax the block is accepted as it is.  Otherwise
// (and always for a row's first visible key, while R.m = kNoMax) the wave
// takes the block max, recomputes P against the new max and returns true: O
// must be rescaled by R.alpha before the next P.V.
template <int D>
__device__ __forceinline__ bool softmax_fix(Rows<D>& R, const f32x16& s, bf16x8* p, float c2,
                                            float ps) {
  if (__ballot(!(ps <= kSumMax)) == 0) {
    R.l += ps;
    R.alpha = 1.f;
    return false;
  }
  float mx = s[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[i]);
  mx = pair_max(mx);
  const float m_new = fmaxf(R.m, mx);
  R.alpha = __builtin_amdgcn_exp2f((R.m - m_new) * c2);
  R.m = m_new;
  R.l = R.l * R.alpha + p_block(s, p, c2, -m_new * c2);
  return true;
}

template <int D>
__device__ __forceinline__ bool softmax_block(Rows<D>& R, const f32x16& s, bf16x8* p, float c2) {
  return softmax_fix<D>(R, s, p, c2, p_block(s, p, c2, -R.m * c2));
}

template <int D>
__device__ __forceinline__ void rescale(Rows<D>& R, float alpha) {
#pragma unroll
  for (int db = 0; db < Geo<D>::NDB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) R.o[db][i] *= alpha;
}

// O^T += V^T P^T over the two 16-key chunks kc = 2kb, 2kb+1 of block kb.
// Chunk kc holds keys 16kc + 4h + r and 16kc + 8 + 4h + r (h = lane >> 5,
// r = 0..3): the key order of the P^T operand taken from the S^T registers.
template <int D>
__device__ __forceinline__ void pv_block(Rows<D>& R, const bf16x8* p, const char* vslot,
                                         const ReadAddr<D>& ra, int kb) {
  constexpr int HALF = (8 / Geo<D>::NI) * Geo<D>::ROWB;   // rows of keys +8
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int db = 0; db < Geo<D>::NDB; ++db) {
      const char* p0 = vslot + (2 * kb + j) * 16 * Geo<D>::ROWB + ra.v[db];
      const bf16x8 vt = tr_read(p0, p0 + HALF);   // kTrRead: keys +8 are HALF further
      R.o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vt, p[j], R.o[db], 0, 0, 0);
    }
}

template <int D>
__device__ __forceinline__ void store_rows(const Rows<D>& R, const HierFwdArgs& a, int head,
                                           int lane, float l_tot, float m) {
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (!R.valid) return;
  uint16_t* op = a.o + (int64_t)R.qtok * a.o_ss + (int64_t)head * a.o_sh;
  const int half = lane >> 5;
#pragma unroll
  for (int db = 0; db < Geo<D>::NDB; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d0 = db * 32 + 8 * g4 + 4 * half;
      u32x2 w;
      w[0] = (uint32_t)f2bf(R.o[db][4 * g4 + 0] * inv) | ((uint32_t)f2bf(R.o[db][4 * g4 + 1] * inv) << 16);
      w[1] = (uint32_t)f2bf(R.o[db][4 * g4 + 2] * inv) | ((uint32_t)f2bf(R.o[db][4 * g4 + 3] * inv) << 16);
      *reinterpret_cast<u32x2*>(op + d0) = w;
    }
  if (a.lse && half == 0) {
    const float lse = l_tot > 0.f ? m * a.scale + __logf(l_tot) : -INFINITY;
    a.lse[(int64_t)head * a.lse_stride_h + R.qtok] = lse;
  }
}

// ---- the kernel ------------------------------------------------------------

template <int D>
struct Ctx {
  const char* gk;
  const char* gv;
  const int32_t* kv_idx;     // tile_kv_idx + kv_off
  const uint32_t* kv_mask;   // tile_kv_mask + kv_off
  const uint32_t* blk;       // tile_blk_and + kv_off / 64
  uint32_t k_ss_b, v_ss_b;
  float c2;
  int nt, wave, lane;
  bool active;
  Copier<D, kRowRead> ck;
  Copier<D, kTrRead> cv;
  ReadAddr<D> ra;
};

// Half-step j = 2t + B of the pipeline: QK of block B of tile t+1 into sq,
// softmax of block j+1 (sc: block 1 of tile t for B = 0, block 0 of tile t+1
// for B = 1) into pn, PV of block B of tile t with pv; then the masks of sq
// (blk_cur: visibility flags of tile t+1).  The three streams are independent,
// so one scheduling region interleaves them: each MFMA is followed by a few
// softmax VALU instructions and the LDS reads of the MFMAs two or three slots
// ahead.  PAR = t & 1 selects the LDS stages: K(t+1) and its masks in PAR^1,
// V(t) in PAR.
template <int D, int PAR, int B>
__device__ __forceinline__ void half_step(Ctx<D>& c, Rows<D>& R, int t, f32x16& sq,
                                          const f32x16& sc, const bf16x8* pv, bf16x8* pn,
                                          bool& resc, float& alpha_pend, uint32_t blk_cur,
                                          const Stages& st) {
  if (resc) rescale<D>(R, alpha_pend);
  sq = qk_block<D>(R.q, st.k[PAR ^ 1], c.ra, B);
  float ps = p_block(sc, pn, c.c2, -R.m * c.c2);
  pv_block<D>(R, pv, st.v[PAR], c.ra, B);
  // NC + 2*NDB MFMAs and NC + 4*NDB LDS reads: three reads per two MFMAs
  constexpr int NM = Geo<D>::NC + 2 * Geo<D>::NDB;
  __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
  for (int i = 0; i < NM; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (i % 2 == 0)
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    else
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);
  }
  // keep the softmax results in this region (otherwise they sink past the
  // branches below, away from the MFMAs they are meant to overlap)
  asm volatile("" : "+v"(pn[0]), "+v"(pn[1]), "+v"(ps));
  resc = softmax_fix<D>(R, sc, pn, c.c2, ps);
  alpha_pend = R.alpha;
  if ((blk_cur & R.bits) != R.bits)
    mask_block(sq, st.m[PAR ^ 1], B, R.qframe, c.lane);
}

// Tile iteration t (t + 1 < nt): copies K(t+2) + masks into stage PAR, runs
// half-step 2t, copies V(t+1) into stage PAR^1, runs half-step 2t+1; the key
// indices and visibility flags of the next iteration are loaded on the way.
// Both stages written are idle for the whole iteration; issuing the copies in
// two bursts keeps a wave from stalling on a full memory queue with all eight
// in flight.  Invariant on entry: K(t+1), masks(t+1) and V(t) resident;
// S(2t+1) (sb) masked; P(2t) (pa) ready with its rescale pending; ik / iv /
// blk hold the indices of tiles min(t+2, nt-1) / t+1 and the flags of tile
// t+1.  Every global load of the iteration is waited for with the copies at
// its end, so nothing inside the half-steps waits on the copies in flight.
template <int D, int PAR>
__device__ __forceinline__ void tile_iter(Ctx<D>& c, Rows<D>& R, int t, f32x16& sa, f32x16& sb,
                                          bf16x8* pa, bf16x8* pb, bool& resc, float& alpha_pend,
                                          Idx<D>& ik, Idx<D>& iv, uint32_t& blk, const Stages& st) {
  if (t + 2 < c.nt) {
    copy_tile<D, kRowRead>(c.gk, c.k_ss_b, c.ck, ik, st.k[PAR], c.wave);
    if (c.wave == 0)
      copy_dwords(c.kv_mask + (t + 2) * kSlab, st.m[PAR], c.lane);
  }
  ik = load_idx<D>(c.kv_idx, min(t + 3, c.nt - 1), c.ck.idx_off);
  const uint32_t blk_pre = c.blk[min(t + 2, c.nt - 1)];
  if (c.active) half_step<D, PAR, 0>(c, R, t, sa, sb, pa, pb, resc, alpha_pend, blk, st);
  copy_tile<D, kTrRead>(c.gv, c.v_ss_b, c.cv, iv, st.v[PAR ^ 1], c.wave);
  iv = load_idx<D>(c.kv_idx, min(t + 2, c.nt - 1), c.ck.idx_off);
  if (c.active) half_step<D, PAR, 1>(c, R, t, sb, sa, pb, pa, resc, alpha_pend, blk, st);
  wait_copies();
  __syncthreads();
  blk = blk_pre;
}

// Last tile (t = nt - 1): softmax of its block 1 (sb) into pb, PV of both
// blocks, then the output rows.
template <int D, int PAR>
__device__ __forceinline__ void tail(Ctx<D>& c, Rows<D>& R, const HierFwdArgs& a, int head,
                                     const f32x16& sb, const bf16x8* pa, bf16x8* pb, bool resc,
                                     float alpha_pend, const Stages& st) {
  const char* vs = st.v[PAR];
  if (resc) rescale<D>(R, alpha_pend);
  resc = softmax_block<D>(R, sb, pb, c.c2);
  alpha_pend = R.alpha;
  pv_block<D>(R, pa, vs, c.ra, 0);
  if (resc) rescale<D>(R, alpha_pend);
  pv_block<D>(R, pb, vs, c.ra, 1);
  store_rows<D>(R, a, head, c.lane, pair_sum(R.l), R.m);
}

// ---- items of at most 32 rows ----------------------------------------------
//
// A hub slot's rows (15 or 18 at n = 3) and the 20-row tail of a 660-row player
// block fill one 32-row sub-block, so in the loop above only wave 0 would
// compute.  Such an item runs the same tile copies (all four waves, same
// stages and barriers), but waves 0 and 1 both take its rows and each
// computes one of the two 32-key blocks of every tile, with its own
// online-softmax state; the two states are merged through LDS at the end.
// Per iteration t a computing wave (block kb = wave) overlaps QK of tile t+1
// with the softmax and P.V of tile t.

template <int D, int PAR>
__device__ __forceinline__ void split_iter(Ctx<D>& c, Rows<D>& R, int t, f32x16& s, Idx<D>& ik,
                                           Idx<D>& iv, uint32_t& blk, const Stages& st) {
  if (t + 2 < c.nt) {
    copy_tile<D, kRowRead>(c.gk, c.k_ss_b, c.ck, ik, st.k[PAR], c.wave);
    if (c.wave == 0)
      copy_dwords(c.kv_mask + (t + 2) * kSlab, st.m[PAR], c.lane);
  }
  ik = load_idx<D>(c.kv_idx, min(t + 3, c.nt - 1), c.ck.idx_off);
  const uint32_t blk_pre = c.blk[min(t + 2, c.nt - 1)];
  copy_tile<D, kTrRead>(c.gv, c.v_ss_b, c.cv, iv, st.v[PAR ^ 1], c.wave);
  iv = load_idx<D>(c.kv_idx, min(t + 2, c.nt - 1), c.ck.idx_off);
  if (c.active) {
    const int kb = c.wave;
    f32x16 sn = qk_block<D>(R.q, st.k[PAR ^ 1], c.ra, kb);
    bf16x8 p[2];
    if (softmax_block<D>(R, s, p, c.c2)) rescale<D>(R, R.alpha);
    pv_block<D>(R, p, st.v[PAR], c.ra, kb);
    if ((blk & R.bits) != R.bits) mask_block(sn, st.m[PAR ^ 1], kb, R.qframe, c.lane);
    s = sn;
  }
  wait_copies();
  __syncthreads();
  blk = blk_pre;
}

// Last tile of a split item, then the merge of the two waves' states: row
// maxima through LDS, then l and O rescaled to the common maximum (O^T as
// fp32 [d-block][element][lane] in the wave's idle K stage), summed by one
// wave per 32-wide d-block.
template <int D, int PAR>
__device__ __forceinline__ void split_tail(Ctx<D>& c, Rows<D>& R, const HierFwdArgs& a, int head,
                                           f32x16& s, const Stages& st) {
  if (c.active) {
    bf16x8 p[2];
    if (softmax_block<D>(R, s, p, c.c2)) rescale<D>(R, R.alpha);
    pv_block<D>(R, p, st.v[PAR], c.ra, c.wave);
  }
  const int q = c.lane & 31;
  float* m_lds = reinterpret_cast<float*>(st.m[0]);
  float* l_lds = reinterpret_cast<float*>(st.m[1]);
  const float l_w = pair_sum(R.l);
  __syncthreads();                 // every wave is done with the stages
  if (c.active && c.lane < 32) m_lds[c.wave * 32 + q] = R.m;
  __syncthreads();
  const float m_tot = fmaxf(m_lds[q], m_lds[32 + q]);
  if (c.active) {
    const float alpha = __builtin_amdgcn_exp2f((R.m - m_tot) * c.c2);
    if (c.lane < 32) l_lds[c.wave * 32 + q] = l_w * alpha;
    float* o_own = reinterpret_cast<float*>(c.wave == 0 ? st.k[0] : st.k[1]);
#pragma unroll
    for (int db = 0; db < Geo<D>::NDB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) o_own[(db * 16 + e) * 64 + c.lane] = R.o[db][e] * alpha;
  }
  __syncthreads();
  if (c.wave >= Geo<D>::NDB) return;
  const float l_tot = l_lds[q] + l_lds[32 + q];
  const int db = c.wave;
  if (!R.valid) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  const float* o0 = reinterpret_cast<const float*>(st.k[0]);
  const float* o1 = reinterpret_cast<const float*>(st.k[1]);
  uint16_t* op = a.o + (int64_t)R.qtok * a.o_ss + (int64_t)head * a.o_sh;
  const int half = c.lane >> 5;
#pragma unroll
  for (int g4 = 0; g4 < 4; ++g4) {
    float v4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = (db * 16 + 4 * g4 + e) * 64 + c.lane;
      v4[e] = (o0[k] + o1[k]) * inv;
    }
    u32x2 w;
    w[0] = (uint32_t)f2bf(v4[0]) | ((uint32_t)f2bf(v4[1]) << 16);
    w[1] = (uint32_t)f2bf(v4[2]) | ((uint32_t)f2bf(v4[3]) << 16);
    *reinterpret_cast<u32x2*>(op + db * 32 + 8 * g4 + 4 * half) = w;
  }
  if (a.lse && db == 0 && half == 0)
    a.lse[(int64_t)head * a.lse_stride_h + R.qtok] =
        l_tot > 0.f ? m_tot * a.scale + __logf(l_tot) : -INFINITY;
}

// Common set-up of both item kinds: the lane's copy and read offsets, the
// item's key list, the first tiles resident in LDS.
template <int D>
__device__ __forceinline__ void item_setup(Ctx<D>& c, const HierFwdArgs& a, const int32_t* it,
                                           int head, int tid, bool active) {
  c.lane = tid & 63;
  c.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kv_off = it[5], kv_cnt = it[6];
  c.nt = kv_cnt / kSlab;
  c.active = active;
  c.c2 = a.scale * 1.4426950408889634f;
  c.gk = reinterpret_cast<const char*>(a.k + (int64_t)head * a.k_sh);
  c.gv = reinterpret_cast<const char*>(a.v + (int64_t)head * a.v_sh);
  c.k_ss_b = (uint32_t)(a.k_ss * 2);
  c.v_ss_b = (uint32_t)(a.v_ss * 2);
  c.kv_idx = a.tile_kv_idx + kv_off;
  c.kv_mask = a.tile_kv_mask + kv_off;
  c.blk = a.tile_blk_and + kv_off / kSlab;
  c.ck.init(c.wave, c.lane);
  c.cv.init(c.wave, c.lane);
  c.ra.init(c.lane);
}

// Prologue copies (nt >= 1): K(0), V(0), K(1) and masks(0, 1) resident; the
// first iteration's indices and flags loaded before the wait.
template <int D>
__device__ __forceinline__ void prologue_copies(Ctx<D>& c, Idx<D>& ik, Idx<D>& iv, uint32_t& blk,
                                                const Stages& st) {
  const int nt = c.nt;
  const Idx<D> i0 = load_idx<D>(c.kv_idx, 0, c.ck.idx_off);
  copy_tile<D, kRowRead>(c.gk, c.k_ss_b, c.ck, i0, st.k[0], c.wave);
  copy_tile<D, kTrRead>(c.gv, c.v_ss_b, c.cv, i0, st.v[0], c.wave);
  if (c.wave == 0) copy_dwords(c.kv_mask, st.m[0], c.lane);
  if (nt > 1) {
    const Idx<D> i1 = load_idx<D>(c.kv_idx, 1, c.ck.idx_off);
    copy_tile<D, kRowRead>(c.gk, c.k_ss_b, c.ck, i1, st.k[1], c.wave);
    if (c.wave == 0) copy_dwords(c.kv_mask + kSlab, st.m[1], c.lane);
  }
  ik = load_idx<D>(c.kv_idx, min(2, nt - 1), c.ck.idx_off);
  iv = load_idx<D>(c.kv_idx, min(1, nt - 1), c.ck.idx_off);
  blk = c.blk[min(1, nt - 1)];
  wait_copies();
  __syncthreads();
}

template <int D>
__device__ __forceinline__ void split_item(const HierFwdArgs& a, const int32_t* it, int head, int tid,
                                        const Stages& st) {
  Ctx<D> c;
  item_setup<D>(c, a, it, head, tid, (tid >> 6) < 2);
  Rows<D> R;
  rows_init<D>(R, a, it, head, 0, c.lane);
  const int nt = c.nt;
  Idx<D> ik, iv;
  uint32_t blk;
  prologue_copies<D>(c, ik, iv, blk, st);
  f32x16 s;
  if (c.active) {
    s = qk_block<D>(R.q, st.k[0], c.ra, c.wave);
    if ((c.blk[0] & R.bits) != R.bits) mask_block(s, st.m[0], c.wave, R.qframe, c.lane);
  }
  __syncthreads();   // every wave has read K stage 0 and masks stage 0
  int t = 0;
  for (; t + 2 < nt; t += 2) {
    split_iter<D, 0>(c, R, t, s, ik, iv, blk, st);
    split_iter<D, 1>(c, R, t + 1, s, ik, iv, blk, st);
  }
  if (t + 1 < nt) {
    split_iter<D, 0>(c, R, t, s, ik, iv, blk, st);
    split_tail<D, 1>(c, R, a, head, s, st);
  } else {
    split_tail<D, 0>(c, R, a, head, s, st);
  }
}

template <int D>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(HierFwdArgs a, int total) {
  __shared__ __align__(16) char lds_k0[Geo<D>::TILEB], lds_k1[Geo<D>::TILEB];
  __shared__ __align__(16) char lds_v0[Geo<D>::TILEB], lds_v1[Geo<D>::TILEB];
  __shared__ __align__(16) char lds_m0[Geo<D>::MBYTES], lds_m1[Geo<D>::MBYTES];
  const Stages st = {{lds_k0, lds_k1}, {lds_v0, lds_v1}, {lds_m0, lds_m1}};
  // XCD-aware mapping: consecutive logical items land on the same XCD (the
  // dispatcher round-robins workgroups over 8 XCDs), so items sharing a head
  // and overlapping key windows share one L2.
  const int logical = hier::xcd_logical(blockIdx.x, gridDim.x);
  if (logical >= total) return;
  const int head = logical / a.n_items;
  const int item = logical - head * a.n_items;
  const int32_t* it = a.tile_items + (int64_t)item * 8;
  const int tid = threadIdx.x;
  const int row_count = it[4];
  if (row_count <= 32 && it[6] >= 2 * kSlab && kSplitSmall) {
    split_item<D>(a, it, head, tid, st);
    return;
  }

  Ctx<D> c;
  item_setup<D>(c, a, it, head, tid, (tid >> 6) * 32 < row_count);
  Rows<D> R;
  rows_init<D>(R, a, it, head, c.wave * 32, c.lane);
  const int nt = c.nt;
  if (nt == 0) {
    if (c.active) store_rows<D>(R, a, head, c.lane, 0.f, -INFINITY);
    return;
  }
  char* const kst0 = st.k[0];
  char* const mst0 = st.m[0];

  // prologue: the first tiles resident; S(0), S(1) (both blocks of tile 0)
  // computed and masked; P(0) from the softmax of S(0)
  Idx<D> ik, iv;
  uint32_t blk;
  prologue_copies<D>(c, ik, iv, blk, st);
  f32x16 sa, sb;
  bf16x8 pa[2], pb[2];
  bool resc = false;
  float alpha_pend = 1.f;
  if (c.active) {
    sa = qk_block<D>(R.q, kst0, c.ra, 0);
    sb = qk_block<D>(R.q, kst0, c.ra, 1);
    if ((c.blk[0] & R.bits) != R.bits) {
      mask_block(sa, mst0, 0, R.qframe, c.lane);
      mask_block(sb, mst0, 1, R.qframe, c.lane);
    }
    resc = softmax_block<D>(R, sa, pa, c.c2);
    alpha_pend = R.alpha;
  }
  __syncthreads();   // every wave has read K stage 0 and masks stage 0

  // steady state, two tile iterations per trip so that every LDS stage offset
  // is a compile-time constant
  int t = 0;
  for (; t + 2 < nt; t += 2) {
    tile_iter<D, 0>(c, R, t, sa, sb, pa, pb, resc, alpha_pend, ik, iv, blk, st);
    tile_iter<D, 1>(c, R, t + 1, sa, sb, pa, pb, resc, alpha_pend, ik, iv, blk, st);
  }
  if (t + 1 < nt) {
    tile_iter<D, 0>(c, R, t, sa, sb, pa, pb, resc, alpha_pend, ik, iv, blk, st);
    if (c.active) tail<D, 1>(c, R, a, head, sb, pa, pb, resc, alpha_pend, st);
  } else {
    if (c.active) tail<D, 0>(c, R, a, head, sb, pa, pb, resc, alpha_pend, st);
  }
}

}  // namespace

extern "C" int hier_attn_fwd(const HierFwdArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  const HierFwdArgs& a = *args;
  HIER_REQUIRE(a.D == 128 || a.D == 64, HIER_EUNSUPPORTED, "head_dim must be 64 or 128, got %d", a.D);
  HIER_REQUIRE(a.H >= 1 && a.n_items >= 0 && a.kv_rows >= 0, HIER_EINVAL,
               "invalid H=%d n_items=%d kv_rows=%d", a.H, a.n_items, a.kv_rows);
  HIER_REQUIRE(a.q && a.k && a.v && a.o && a.tile_items && a.tile_kv_idx && a.tile_kv_mask &&
                   a.tile_blk_and,
               HIER_EINVAL, "NULL tensor pointer");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  HIER_REQUIRE(al16(a.q) && al16(a.k) && al16(a.v) && al16(a.o) && al16(a.tile_kv_idx),
               HIER_EINVAL, "q/k/v/o and the key index list must be 16-byte aligned");
  HIER_REQUIRE(a.q_ss % 8 == 0 && a.q_sh % 8 == 0 && a.k_ss % 8 == 0 && a.k_sh % 8 == 0 &&
                   a.v_ss % 8 == 0 && a.v_sh % 8 == 0 && a.o_ss % 4 == 0 && a.o_sh % 4 == 0,
               HIER_EINVAL, "strides must keep 16-byte rows aligned");
  HIER_REQUIRE(a.k_ss >= 0 && a.k_sh >= 0 && a.v_ss >= 0 && a.v_sh >= 0, HIER_EINVAL,
               "K/V strides must be non-negative");
  // K / V rows are addressed with 32-bit byte offsets from k / v.
  const __int128 k_ext = hier::span_bytes(a.kv_rows, a.k_ss, a.k_sh, a.H, a.D);
  const __int128 v_ext = hier::span_bytes(a.kv_rows, a.v_ss, a.v_sh, a.H, a.D);
  HIER_REQUIRE(k_ext <= ((__int128)1 << 32) && v_ext <= ((__int128)1 << 32), HIER_EUNSUPPORTED,
               "K/V views must span at most 4 GiB");
  HIER_REQUIRE(copy_rows_ok(a.kv_rows, a.k_ss) && copy_rows_ok(a.kv_rows, a.v_ss),
               HIER_EUNSUPPORTED, "K/V need at most 2^24 rows and a row stride under 8M elements");
  if (a.n_items == 0) return HIER_OK;
  const int64_t total = (int64_t)a.n_items * a.H;
  HIER_REQUIRE(total <= hier::kMaxLaunchItems, HIER_EUNSUPPORTED, "too many work items");
  const int grid = (int)hier::xcd_grid(total);
  if (a.D == 128)
    hipLaunchKernelGGL(attn_fwd_kernel<128>, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, a,
                       (int)total);
  else
    hipLaunchKernelGGL(attn_fwd_kernel<64>, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, a,
                       (int)total);
  return hier::check_launch("attn_fwd_kernel");
}
