// Segmented-metadata builder: hierarchical membership -> key lists / tile lists.
//
// One workgroup per (temporal block, query stream).  A stream is one player,
// one local-hub slot or the global hub; its segments are the stream's rows of
// each query frame of the block.  Every key list of the reference is a
// concatenation of whole cached frames ("runs"), and the run order of a stream
// does not depend on the query frame -- only each run's `allowed` flag does.
// So the workgroup enumerates the stream's runs once, evaluates the edge rule
// per (run, query frame) into a bitmask, and from those masks
//
//   * counts and writes the compact key lists of _build_metadata
//     (multics/models/kernels/hier_segmented_attention.py:156-395),
//   * counts and writes the Tiled128 chunk layout of _pack_layout and the
//     cached / full-sequence dense slot orders
//     (multics/models/kernels/hier_tiled_attention.py:182-241, 244-429, 474-655),
//   * writes this library's attention tile list: the ordered union of the
//     stream's key lists with a per-key bitmask over query frames, plus the
//     AND of those masks per 64 keys and the work-item descriptors.
//
// Integer work only; HBM-bound and tiny (a few MB per topology).
#include "hier_common.h"

#include <algorithm>
#include <climits>

namespace {

constexpr int kThreads = 256;
constexpr int kMaxRuns = 1024;     // cached frame runs per stream
constexpr int kMaxChunks = 2048;   // Tiled128 dense chunks per segment
constexpr int kTiledN = 128;       // hier_tiled_attention.py:33
constexpr int kTiledM = 16;        // hier_tiled_attention.py:32
constexpr int kTileKeys = 64;      // attention kernel key-tile width

struct Topo {
  const HierTopo* t;
  int b;        // block
  int fa, fl, fg;
};

enum RunType { kAgent = 0, kLocal = 1, kGlobal = 2 };

struct Run {
  int type;
  int sid;      // player / group / 0
  int fi;       // frame index inside the cached stream
  int kf;       // absolute frame id
  int width;
  bool present; // part of the Tiled128 dense list
  int sub;      // 0 own/plain, 1 direct
};

__device__ __forceinline__ bool temporal_ok(int qf, int kf, int nb, int w) {
  // hier_segmented_attention.py:117-122 (frames are non-negative).
  if (kf / nb > qf / nb) return false;
  return w == -1 || (qf - kf) < w;
}

__device__ __forceinline__ int stream_kind(const HierTopo& t, int s) {
  if (s < t.P) return kAgent;
  if (s < t.P + t.N) return kLocal;
  return kGlobal;
}

__device__ __forceinline__ int num_runs(const Topo& c, int kind) {
  const HierTopo& t = *c.t;
  int nl = t.no_local ? 0 : 1;
  if (kind == kAgent)
    return c.fa + (t.direct ? (t.P - 1) * t.n_frames : 0) + nl * t.N * c.fl + c.fg;
  if (kind == kLocal) return t.P * c.fa + c.fl + c.fg;
  return nl * t.N * c.fl + c.fg + t.P * c.fa;
}

__device__ __forceinline__ int agent_frame(const Topo& c, int p, int fi) {
  return c.t->agent_frames[((int64_t)c.b * c.t->P + p) * c.t->fa_max + fi];
}
__device__ __forceinline__ int local_frame(const Topo& c, int g, int fi) {
  return c.t->local_frames[((int64_t)c.b * c.t->N + g) * c.t->fl_max + fi];
}
__device__ __forceinline__ int global_frame(const Topo& c, int fi) {
  return c.t->global_frames[(int64_t)c.b * c.t->fg_max + fi];
}
__device__ __forceinline__ int q_frame(const Topo& c, int j) {
  return c.t->q_frames[(int64_t)c.b * c.t->n_frames + j];
}

__device__ Run decode(const Topo& c, int kind, int s, int r) {
  const HierTopo& t = *c.t;
  Run u{};
  u.sub = 0;
  if (kind == kAgent) {
    int p = s;
    if (r < c.fa) {
      u.type = kAgent; u.sid = p; u.fi = r; u.present = true;
    } else {
      r -= c.fa;
      int dn = t.direct ? (t.P - 1) * t.n_frames : 0;
      if (r < dn) {
        int oi = r / t.n_frames, kr = r % t.n_frames;
        int o = oi + (oi >= p ? 1 : 0);
        int kf = q_frame(c, kr);
        int fi = 0;
        for (int i = 0; i < c.fa; ++i)
          if (agent_frame(c, o, i) == kf) { fi = i; break; }
        u.type = kAgent; u.sid = o; u.fi = fi; u.present = true; u.sub = 1;
      } else {
        r -= dn;
        int nloc = t.no_local ? 0 : t.N * c.fl;
        if (r < nloc) {
          u.type = kLocal; u.sid = r / c.fl; u.fi = r % c.fl; u.present = true;
        } else {
          u.type = kGlobal; u.sid = 0; u.fi = r - nloc; u.present = false;
        }
      }
    }
  } else if (kind == kLocal) {
    if (r < t.P * c.fa) {
      u.type = kAgent; u.sid = r / c.fa; u.fi = r % c.fa;
    } else if (r < t.P * c.fa + c.fl) {
      u.type = kLocal; u.sid = s - t.P; u.fi = r - t.P * c.fa;
    } else {
      u.type = kGlobal; u.sid = 0; u.fi = r - t.P * c.fa - c.fl;
    }
    u.present = true;
  } else {
    int nloc = t.no_local ? 0 : t.N * c.fl;
    if (r < nloc) {
      u.type = kLocal; u.sid = r / c.fl; u.fi = r % c.fl; u.present = true;
    } else if (r < nloc + c.fg) {
      u.type = kGlobal; u.sid = 0; u.fi = r - nloc; u.present = true;
    } else {
      r -= nloc + c.fg;
      u.type = kAgent; u.sid = r / c.fa; u.fi = r % c.fa; u.present = false;
    }
  }
  if (u.type == kAgent) { u.kf = agent_frame(c, u.sid, u.fi); u.width = t.L; }
  else if (u.type == kLocal) { u.kf = local_frame(c, u.sid, u.fi); u.width = t.KL; }
  else { u.kf = global_frame(c, u.fi); u.width = t.KG; }
  return u;
}

__device__ __forceinline__ bool mem_at(const HierTopo& t, int f, int g, int p) {
  return t.membership[((int64_t)f * t.N + g) * t.P + p] != 0;
}
__device__ __forceinline__ bool go_at(const HierTopo& t, int f, int p) {
  return t.global_only[(int64_t)f * t.P + p] != 0;
}
__device__ __forceinline__ int label_at(const Topo& c, int j, int p) {
  return c.t->labels[((int64_t)c.b * c.t->n_frames + j) * c.t->P + p];
}
__device__ __forceinline__ bool qactive_at(const Topo& c, int j, int g) {
  return c.t->q_active[((int64_t)c.b * c.t->n_frames + j) * c.t->N + g] != 0;
}
__device__ __forceinline__ bool lactive_at(const Topo& c, int g, int fi) {
  return c.t->local_active[((int64_t)c.b * c.t->N + g) * c.t->fl_max + fi] != 0;
}

// Edge rule of one run for query frame j (cached-SDPA semantics,
// hier_segmented_attention.py:276-368; attention.py:797-996).
__device__ bool allowed(const Topo& c, int kind, int s, const Run& u, int j) {
  const HierTopo& t = *c.t;
  int qf = q_frame(c, j);
  bool tmp = temporal_ok(qf, u.kf, t.n_block, t.local_attn);
  if (kind == kAgent) {
    int p = s;
    if (u.type == kAgent) {
      if (u.sub == 0) return tmp;
      int o = u.sid;
      bool share;
      if (t.use_membership) {
        share = false;
        for (int g = 0; g < t.N; ++g) share |= mem_at(t, qf, g, p) && mem_at(t, qf, g, o);
      } else {
        share = label_at(c, j, o) == label_at(c, j, p);
      }
      return share && (u.kf / t.n_block == qf / t.n_block);
    }
    if (u.type == kLocal) {
      int g = u.sid;
      bool own = t.use_membership ? mem_at(t, qf, g, p) : (label_at(c, j, p) == g);
      return own && lactive_at(c, g, u.fi) && tmp;
    }
    if (t.KG <= 0) return false;
    return (t.no_local || (t.use_membership && go_at(t, qf, p))) && tmp;
  }
  if (kind == kLocal) {
    int g = s - t.P;
    if (!qactive_at(c, j, g)) return false;
    if (u.type == kAgent) {
      int p = u.sid;
      bool in = t.use_membership ? mem_at(t, qf, g, p) : (label_at(c, j, p) == g);
      return in && tmp;
    }
    if (u.type == kLocal) return lactive_at(c, g, u.fi) && tmp;
    return tmp;
  }
  // global rows
  if (u.type == kLocal) return lactive_at(c, u.sid, u.fi) && tmp;
  if (u.type == kGlobal) return tmp;
  if (t.no_local) return tmp;
  if (t.use_membership) return go_at(t, u.kf, u.sid) && tmp;
  return false;
}

__device__ __forceinline__ int ref_base(const Topo& c, const Run& u) {
  const HierTopo& t = *c.t;
  if (u.type == kAgent) return t.ref_agent_base[((int64_t)c.b * t.P + u.sid) * t.fa_max + u.fi];
  if (u.type == kLocal) return t.ref_local_base[((int64_t)c.b * t.N + u.sid) * t.fl_max + u.fi];
  return t.ref_global_base[(int64_t)c.b * t.fg_max + u.fi];
}
__device__ __forceinline__ int tile_base(const Topo& c, const Run& u) {
  const HierTopo& t = *c.t;
  if (u.type == kAgent) return t.tile_agent_base[((int64_t)c.b * t.P + u.sid) * t.fa_max + u.fi];
  if (u.type == kLocal) return t.tile_local_base[((int64_t)c.b * t.N + u.sid) * t.fl_max + u.fi];
  return t.tile_global_base[(int64_t)c.b * t.fg_max + u.fi];
}

__device__ __forceinline__ int seg_id(const HierTopo& t, int kind, int s, int j) {
  int n = t.n_frames;
  if (kind == kAgent) return s * n + j;
  if (kind == kLocal) return t.P * n + j * t.N + (s - t.P);
  return t.P * n + (t.no_local ? 0 : n * t.N) + j;
}

__device__ __forceinline__ int qlen_of(const HierTopo& t, int kind) {
  return kind == kAgent ? t.L : (kind == kLocal ? t.KL : t.KG);
}

// Number of programs before segment `sid` when every segment is split into
// block_m-row programs (hier_segmented_attention.py:381-384).
__device__ __forceinline__ int64_t prog_before(const HierTopo& t, int sid, int bm) {
  auto cl = [bm](int x) { return (int64_t)((x + bm - 1) / bm); };
  int np = t.P * t.n_frames;
  int nlo = t.no_local ? 0 : t.n_frames * t.N;
  if (sid < np) return sid * cl(t.L);
  if (sid < np + nlo) return np * cl(t.L) + (sid - np) * cl(t.KL);
  return np * cl(t.L) + nlo * cl(t.KL) + (int64_t)(sid - np - nlo) * cl(t.KG);
}

// ---- workgroup scan helpers (256 threads = 4 waves of 64) -----------------

__device__ __forceinline__ int wave_incl_scan(int v) {
  int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// Exclusive scan of one value per thread; returns the prefix, *total the sum.
__device__ int block_excl_scan(int v, int* tmp4, int* total) {
  int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int inc = wave_incl_scan(v);
  __syncthreads();
  if (lane == 63) tmp4[w] = inc;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) {
    int x = tmp4[i];
    base += (i < w) ? x : 0;
    tot += x;
  }
  *total = tot;
  return base + inc - v;
}

// In-LDS exclusive prefix of vals[0..n) into out[0..n]; out[n] = total.
__device__ int lds_excl_prefix(const int* vals, int* out, int n, int* tmp4) {
  int per = (n + kThreads - 1) / kThreads;
  int lo = threadIdx.x * per, hi = min(lo + per, n);
  int sum = 0;
  for (int i = lo; i < hi; ++i) sum += vals[i];
  int total;
  int base = block_excl_scan(sum, tmp4, &total);
  for (int i = lo; i < hi; ++i) {
    out[i] = base;
    base += vals[i];
  }
  if (threadIdx.x == 0) out[n] = total;
  __syncthreads();
  return total;
}

// Largest r in [0, n) with off[r] <= x (off has n+1 non-decreasing entries).
__device__ __forceinline__ int find_run(const int* off, int n, int x) {
  int lo = 0, hi = n;  // answer in [lo, hi)
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if (off[mid] <= x) lo = mid; else hi = mid;
  }
  return lo;
}

struct Shared {
  uint32_t mask[kMaxRuns];
  int width[kMaxRuns];
  int val[kMaxRuns];
  int off[kMaxRuns + 1];
  int doff[kMaxRuns + 1];
  int chunk[kMaxChunks + 1];
  int kept[kMaxChunks];
  int cflag[kMaxChunks];
  int tmp4[4];
};

__device__ void eval_masks(const Topo& c, int kind, int s, int R, Shared& sh) {
  for (int r = threadIdx.x; r < R; r += kThreads) {
    Run u = decode(c, kind, s, r);
    uint32_t m = 0;
    for (int j = 0; j < c.t->n_frames; ++j)
      if (u.width > 0 && allowed(c, kind, s, u, j)) m |= 1u << j;
    sh.mask[r] = m;
    sh.width[r] = u.width;
  }
  __syncthreads();
}

// Mark the Tiled128 chunks that hold an allowed slot of query frame j; returns
// the number of kept chunks, with sh.chunk[c] = position of chunk c among kept.
__device__ int mark_chunks(const Topo& c, int kind, int s, int R, int j, int dense_total,
                           Shared& sh) {
  int nch = (dense_total + kTiledN - 1) / kTiledN;
  for (int i = threadIdx.x; i < nch; i += kThreads) sh.cflag[i] = 0;
  __syncthreads();
  for (int r = threadIdx.x; r < R; r += kThreads) {
    int w = sh.doff[r + 1] - sh.doff[r];
    if (w > 0 && ((sh.mask[r] >> j) & 1u)) {
      for (int ch = sh.doff[r] / kTiledN; ch <= (sh.doff[r] + w - 1) / kTiledN; ++ch)
        sh.cflag[ch] = 1;  // benign identical writes
    }
  }
  __syncthreads();
  int kept = lds_excl_prefix(sh.cflag, sh.chunk, nch, sh.tmp4);
  return kept;
}

__device__ void dense_offsets(const Topo& c, int kind, int s, int R, Shared& sh, int* total) {
  for (int r = threadIdx.x; r < R; r += kThreads) {
    Run u = decode(c, kind, s, r);
    sh.val[r] = u.present ? u.width : 0;
  }
  __syncthreads();
  *total = lds_excl_prefix(sh.val, sh.doff, R, sh.tmp4);
}

__global__ __launch_bounds__(kThreads) void meta_count_kernel(HierTopo t, HierMetaCounts out) {
  __shared__ Shared sh;
  const int NS = t.P + t.N + 1;
  Topo c;
  c.t = &t;
  c.b = blockIdx.x / NS;
  const int s = blockIdx.x % NS;
  c.fa = t.fa[c.b]; c.fl = t.no_local ? 0 : t.fl[c.b]; c.fg = t.fg[c.b];
  const int kind = stream_kind(t, s);
  if (kind == kLocal && t.no_local) return;
  const int R = num_runs(c, kind);
  const int n = t.n_frames;
  const int n_seg = n * (t.P + (t.no_local ? 0 : t.N) + 1);
  eval_masks(c, kind, s, R, sh);

  // union of the stream's key lists
  for (int r = threadIdx.x; r < R; r += kThreads) sh.val[r] = sh.mask[r] ? sh.width[r] : 0;
  __syncthreads();
  int uni = lds_excl_prefix(sh.val, sh.off, R, sh.tmp4);
  if (threadIdx.x == 0)
    out.tile_count[(int64_t)c.b * NS + s] = (uni + kTileKeys - 1) / kTileKeys * kTileKeys;

  int dense_total = 0;
  dense_offsets(c, kind, s, R, sh, &dense_total);
  for (int j = 0; j < n; ++j) {
    int cnt = 0, logical = 0;
    for (int r = threadIdx.x; r < R; r += kThreads) {
      if ((sh.mask[r] >> j) & 1u) {
        cnt += sh.width[r];
        logical += sh.doff[r + 1] - sh.doff[r];
      }
    }
    int tot_cnt, tot_log;
    block_excl_scan(cnt, sh.tmp4, &tot_cnt);
    __syncthreads();
    block_excl_scan(logical, sh.tmp4, &tot_log);
    int kept = mark_chunks(c, kind, s, R, j, dense_total, sh);
    if (threadIdx.x == 0) {
      int64_t o = (int64_t)c.b * n_seg + seg_id(t, kind, s, j);
      out.seg_count[o] = tot_cnt;
      out.logical_count[o] = tot_log;
      out.dense_count[o] = dense_total;
      out.tiled_count[o] = kept * kTiledN;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(kThreads) void meta_build_kernel(HierTopo t, HierMetaOut out) {
  __shared__ Shared sh;
  const int NS = t.P + t.N + 1;
  Topo c;
  c.t = &t;
  c.b = blockIdx.x / NS;
  const int s = blockIdx.x % NS;
  c.fa = t.fa[c.b]; c.fl = t.no_local ? 0 : t.fl[c.b]; c.fg = t.fg[c.b];
  const int kind = stream_kind(t, s);
  if (kind == kLocal && t.no_local) return;
  const int R = num_runs(c, kind);
  const int n = t.n_frames;
  const int qlen = qlen_of(t, kind);
  const int tix = kind == kAgent ? 0 : (kind == kLocal ? 1 : 2);
  eval_masks(c, kind, s, R, sh);

  // ---- attention tile list --------------------------------------------------
  if (out.tile_kv_idx) {
    for (int r = threadIdx.x; r < R; r += kThreads) sh.val[r] = sh.mask[r] ? sh.width[r] : 0;
    __syncthreads();
    int uni = lds_excl_prefix(sh.val, sh.off, R, sh.tmp4);
    int padded = (uni + kTileKeys - 1) / kTileKeys * kTileKeys;
    int64_t base = out.tile_kv_off[(int64_t)c.b * NS + s];
    int pad_idx = 0;
    if (uni > 0) {
      int r0 = find_run(sh.off, R, 0);
      pad_idx = tile_base(c, decode(c, kind, s, r0));
    }
    for (int i = threadIdx.x; i < padded; i += kThreads) {
      int idx = pad_idx;
      uint32_t m = 0;
      if (i < uni) {
        int r = find_run(sh.off, R, i);
        idx = tile_base(c, decode(c, kind, s, r)) + (i - sh.off[r]);
        m = sh.mask[r];
      }
      out.tile_kv_idx[base + i] = idx;
      out.tile_kv_mask[base + i] = m;
    }
    for (int k = threadIdx.x; k < padded / kTileKeys; k += kThreads) {
      uint32_t a = ~0u;
      int i0 = k * kTileKeys;
      if (i0 + kTileKeys > uni) {
        a = 0;
      } else {
        int r = find_run(sh.off, R, i0);
        while (r < R && sh.off[r] < i0 + kTileKeys) {
          if (sh.off[r + 1] > sh.off[r]) a &= sh.mask[r];
          ++r;
        }
      }
      out.tile_blk_and[base / kTileKeys + k] = a;
    }
    if (out.tile_items) {
      int rows = n * qlen;
      int rpi = out.rows_per_item;
      int nit = (rows + rpi - 1) / rpi;
      int64_t it0 = out.tile_item_off[(int64_t)c.b * NS + s];
      for (int it = threadIdx.x; it < nit; it += kThreads) {
        int32_t* d = out.tile_items + (it0 + it) * 8;
        d[0] = t.tile_qbase[(int64_t)c.b * NS + s];
        d[1] = t.tile_qstride[tix];
        d[2] = qlen;
        d[3] = it * rpi;
        d[4] = min(rpi, rows - it * rpi);
        d[5] = (int32_t)base;
        d[6] = padded;
        d[7] = n;
      }
    }
    __syncthreads();
  }

  // ---- _build_metadata arrays -----------------------------------------------
  if (out.seg_kv_index) {
    const int n_seg = n * (t.P + (t.no_local ? 0 : t.N) + 1);
    const int max_k = out.seg_max_k[c.b];
    const int bm = out.block_m;
    for (int j = 0; j < n; ++j) {
      for (int r = threadIdx.x; r < R; r += kThreads)
        sh.val[r] = ((sh.mask[r] >> j) & 1u) ? sh.width[r] : 0;
      __syncthreads();
      int cnt = lds_excl_prefix(sh.val, sh.off, R, sh.tmp4);
      int sid = seg_id(t, kind, s, j);
      int64_t row = out.seg_kv_off[c.b] + (int64_t)sid * max_k;
      for (int i = threadIdx.x; i < max_k; i += kThreads) {
        int v = 0;
        if (i < cnt) {
          int r = find_run(sh.off, R, i);
          v = ref_base(c, decode(c, kind, s, r)) + (i - sh.off[r]);
        }
        out.seg_kv_index[row + i] = v;
      }
      if (threadIdx.x == 0) out.seg_kv_count[(int64_t)c.b * n_seg + sid] = cnt;
      int qstart = t.ref_qbase[(int64_t)c.b * NS + s] + j * t.ref_qstride[tix];
      int np = (qlen + bm - 1) / bm;
      int64_t p0 = out.seg_prog_off[c.b] + prog_before(t, sid, bm);
      for (int k = threadIdx.x; k < np; k += kThreads) {
        out.seg_prog_qbase[p0 + k] = qstart + k * bm;
        out.seg_prog_nq[p0 + k] = min(bm, qlen - k * bm);
        out.seg_prog_seg[p0 + k] = sid;
      }
      __syncthreads();
    }
  }

  // ---- Tiled128 arrays (labels form only) ----------------------------------
  if (out.tiled_kv_index && !t.use_membership && !t.no_local) {
    const int n_seg = n * (t.P + t.N + 1);
    const int max_k = out.tiled_max_k[c.b];
    int dense_total = 0;
    dense_offsets(c, kind, s, R, sh, &dense_total);
    for (int j = 0; j < n; ++j) {
      int kept = mark_chunks(c, kind, s, R, j, dense_total, sh);
      int nch = (dense_total + kTiledN - 1) / kTiledN;
      for (int ch = threadIdx.x; ch < nch; ch += kThreads)
        if (sh.cflag[ch]) sh.kept[sh.chunk[ch]] = ch;
      __syncthreads();
      int sid = seg_id(t, kind, s, j);
      int64_t row = out.tiled_kv_off[c.b] + (int64_t)sid * max_k;
      for (int i = threadIdx.x; i < max_k; i += kThreads) {
        int v = 0;
        uint8_t ok = 0;
        if (i < kept * kTiledN) {
          int slot = sh.kept[i / kTiledN] * kTiledN + (i % kTiledN);
          if (slot < dense_total) {
            int r = find_run(sh.doff, R, slot);
            v = ref_base(c, decode(c, kind, s, r)) + (slot - sh.doff[r]);
            ok = (sh.mask[r] >> j) & 1u;
          }
        }
        out.tiled_kv_index[row + i] = v;
        out.tiled_kv_valid[row + i] = ok;
      }
      if (threadIdx.x == 0) out.tiled_kv_count[(int64_t)c.b * n_seg + sid] = kept * kTiledN;
      int qstart = t.ref_qbase[(int64_t)c.b * NS + s] + j * t.ref_qstride[tix];
      int np = (qlen + kTiledM - 1) / kTiledM;
      int64_t p0 = out.tiled_prog_off[c.b] + prog_before(t, sid, kTiledM);
      for (int k = threadIdx.x; k < np; k += kThreads) {
        out.tiled_prog_qbase[p0 + k] = qstart + k * kTiledM;
        out.tiled_prog_nq[p0 + k] = min(kTiledM, qlen - k * kTiledM);
        out.tiled_prog_seg[p0 + k] = sid;
      }
      __syncthreads();
    }
  }
}

int validate(const HierTopo* t) {
  HIER_REQUIRE(t != nullptr, HIER_EINVAL, "topology is NULL");
  HIER_REQUIRE(t->P >= 1 && t->N >= 1 && t->L >= 1 && t->KL >= 0 && t->KG >= 0, HIER_EINVAL,
               "invalid sizes P=%d N=%d L=%d KL=%d KG=%d", t->P, t->N, t->L, t->KL, t->KG);
  HIER_REQUIRE(t->n_frames >= 1 && t->n_frames <= 32, HIER_EUNSUPPORTED,
               "n_frames must be in [1,32], got %d", t->n_frames);
  HIER_REQUIRE(t->n_block >= 1, HIER_EINVAL, "n_block must be >= 1");
  HIER_REQUIRE(t->B >= 1, HIER_EINVAL, "B must be >= 1");
  HIER_REQUIRE(t->fa_max >= 0 && t->fl_max >= 0 && t->fg_max >= 0, HIER_EINVAL,
               "invalid frame pitches fa_max=%d fl_max=%d fg_max=%d", t->fa_max, t->fl_max,
               t->fg_max);
  // bounds that keep every size product below in 64 bits (the run bound
  // below implies P, N, fa_max, fl_max, fg_max <= kMaxRuns + 1 anyway)
  HIER_REQUIRE(t->P <= kMaxRuns + 1 && t->N <= kMaxRuns + 1 && t->fa_max <= kMaxRuns &&
                   t->fl_max <= kMaxRuns && t->fg_max <= kMaxRuns && t->L <= (1 << 20) &&
                   t->KL <= (1 << 20) && t->KG <= (1 << 20) && t->B <= (1 << 20),
               HIER_EUNSUPPORTED, "topology too large (P=%d N=%d L=%d B=%d)", t->P, t->N, t->L,
               t->B);
  HIER_REQUIRE((int64_t)t->B * (t->P + t->N + 1) <= INT32_MAX, HIER_EUNSUPPORTED,
               "too many (block, stream) groups");
  HIER_REQUIRE(!t->no_local || t->KL == 0, HIER_EINVAL, "no_local requires K_L=0");
  HIER_REQUIRE(t->fa && t->fl && t->fg && t->agent_frames && t->global_frames && t->q_frames &&
                   t->q_active && t->ref_agent_base && t->ref_global_base &&
                   t->tile_agent_base && t->tile_global_base && t->ref_qbase && t->tile_qbase,
               HIER_EINVAL, "topology array pointer is NULL");
  HIER_REQUIRE(t->use_membership ? (t->membership && t->global_only) : (t->labels != nullptr),
               HIER_EINVAL, "membership/global_only or labels missing");
  HIER_REQUIRE(t->no_local || (t->local_frames && t->local_active && t->ref_local_base &&
                               t->tile_local_base),
               HIER_EINVAL, "local stream arrays missing");
  int NS = t->P + t->N + 1;
  int64_t rmax = (int64_t)t->P * t->fa_max + (int64_t)t->N * t->fl_max + t->fg_max +
                 (int64_t)(t->P - 1) * t->n_frames;
  HIER_REQUIRE(rmax <= kMaxRuns, HIER_EUNSUPPORTED, "too many cached frame runs (%lld > %d)",
               (long long)rmax, kMaxRuns);
  int64_t dmax = (int64_t)t->P * t->fa_max * t->L + (int64_t)t->N * t->fl_max * t->KL +
                 (int64_t)t->fg_max * t->KG + (int64_t)t->P * t->n_frames * t->L;
  HIER_REQUIRE(dmax <= (int64_t)kMaxChunks * kTiledN, HIER_EUNSUPPORTED,
               "dense slot list too long (%lld)", (long long)dmax);
  (void)NS;
  return HIER_OK;
}

}  // namespace

extern "C" int hier_meta_count(const HierTopo* topo, const HierMetaCounts* counts, void* stream) {
  hier::clear_error();
  int rc = validate(topo);
  if (rc) return rc;
  HIER_REQUIRE(counts && counts->seg_count && counts->tiled_count && counts->dense_count &&
                   counts->logical_count && counts->tile_count,
               HIER_EINVAL, "count output pointer is NULL");
  int grid = topo->B * (topo->P + topo->N + 1);
  hipLaunchKernelGGL(meta_count_kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream,
                     *topo, *counts);
  return hier::check_launch("meta_count_kernel");
}

extern "C" int hier_meta_build(const HierTopo* topo, const HierMetaOut* out, void* stream) {
  hier::clear_error();
  int rc = validate(topo);
  if (rc) return rc;
  HIER_REQUIRE(out != nullptr, HIER_EINVAL, "output descriptor is NULL");
  if (out->tile_kv_idx)
    HIER_REQUIRE(out->tile_kv_mask && out->tile_blk_and && out->tile_kv_off, HIER_EINVAL,
                 "tile list arrays incomplete");
  if (out->tile_items)
    HIER_REQUIRE(out->tile_item_off && out->rows_per_item > 0 && out->rows_per_item % 32 == 0,
                 HIER_EINVAL, "work item arguments invalid");
  if (out->seg_kv_index)
    HIER_REQUIRE(out->seg_kv_count && out->seg_prog_qbase && out->seg_prog_nq &&
                     out->seg_prog_seg && out->seg_prog_off && out->seg_kv_off &&
                     out->seg_max_k && out->block_m > 0,
                 HIER_EINVAL, "segmented arrays incomplete");
  if (out->tiled_kv_index)
    HIER_REQUIRE(out->tiled_kv_valid && out->tiled_kv_count && out->tiled_prog_qbase &&
                     out->tiled_prog_nq && out->tiled_prog_seg && out->tiled_prog_off &&
                     out->tiled_kv_off && out->tiled_max_k,
                 HIER_EINVAL, "tiled arrays incomplete");
  int grid = topo->B * (topo->P + topo->N + 1);
  hipLaunchKernelGGL(meta_build_kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream,
                     *topo, *out);
  return hier::check_launch("meta_build_kernel");
}

// ---- backward lists derived from a full-sequence tile list -----------------
//
// The dK / dV passes of the backward walk a key-major list and the membership
// STE pass a list of the membership-gated edges; both follow from the forward
// tile list alone.  In a full-sequence topology every token is a query row of
// exactly one (block, stream) group (the items that share one key list) and a
// key of the same group, and a group's key list is a concatenation of whole
// key frames ("runs") of groups, each run with one bitmask over the query
// group's frames.
//
//   key-major list of key group G: the query units (g, j) -- query group g,
//     its frame j -- that see any frame of G, in (g, j) order, each unit's
//     qlen(g) rows with the bitmask over G's frames it sees; padded to 64
//     with (row 0, mask 0).  Items: the forward items with the key offset /
//     count of their group's list.
//   STE list of group g: player groups keep their local-hub keys (class =
//     group), local-hub groups their player keys (class = player), in list
//     order stably grouped by class, padded to 64; global-hub groups and
//     groups without such a key are dropped.
//
// Pass 1 (hier_derive_count) maps tokens to groups, collects the runs into a
// dense [key group][query group][query frame] table of key-frame bitmasks,
// counts both lists and prefix-sums their offsets; the caller reads back the
// totals (entries, pairs, error flags) to size pass 2 (hier_derive_build),
// which writes the lists, the per-64-key ANDs of the masks and the items.

namespace {

constexpr int kDeriveThreads = 256;
constexpr int kScanThreads = 1024;
constexpr int kClasses = 64;            // STE classes (players or groups, <= 62)
constexpr int64_t kMaxTable = 1ll << 26;  // n_groups^2 * nq_max table entries
constexpr int kRunSplit = 8;            // workgroups per group list in the runs pass

enum DeriveErr {
  kErrTwoGroups = 1,      // a token is a query row of two groups
  kErrNoGroup = 2,        // a key is not a query row of any group
  kErrRuns = 4,           // key lists are not whole key frames
  kErrItems = 8,          // items are not grouped / frames exceed nq_max
  kErrOverflow = 16       // a list offset does not fit in int32
};

struct DeriveWs {
  int32_t* grp_of_item;   // [n_items]
  int32_t* grp_first;     // [n_groups + 1]
  int32_t* tok_g;         // [rows]
  int32_t* tok_r;         // [rows]
  uint32_t* table;        // [n_groups][n_groups][nq]: (key group G, query group g, frame j)
  int32_t* runs;          // [n_groups][n_groups][nq]: runs of (query g, key group G, key frame f)
  int32_t* t_size;        // [n_groups] padded key-major list sizes
  int64_t* t_off;         // [n_groups + 1]
  int32_t* s_cnt;         // [n_groups][kClasses]
  int32_t* s_size;        // [n_groups] padded STE list sizes
  int64_t* s_off;         // [n_groups + 1]
  int64_t* s_item_off;    // [n_groups + 1]
};

__host__ __device__ inline int64_t al256(int64_t b) { return (b + 255) & ~(int64_t)255; }

__host__ __device__ inline int64_t derive_ws_layout(const HierDeriveArgs& a, DeriveWs* w) {
  const int64_t ng = a.n_groups, tab = ng * ng * a.nq_max;
  int64_t o = 0;
  char* base = reinterpret_cast<char*>(a.ws);
  auto take = [&](int64_t bytes) { char* p = base ? base + o : nullptr; o += al256(bytes); return p; };
  DeriveWs d;
  d.grp_of_item = reinterpret_cast<int32_t*>(take(4 * (int64_t)a.n_items));
  d.grp_first = reinterpret_cast<int32_t*>(take(4 * (ng + 1)));
  d.tok_g = reinterpret_cast<int32_t*>(take(4 * (int64_t)a.rows));
  d.tok_r = reinterpret_cast<int32_t*>(take(4 * (int64_t)a.rows));
  d.table = reinterpret_cast<uint32_t*>(take(4 * tab));
  d.runs = reinterpret_cast<int32_t*>(take(4 * tab));
  d.t_size = reinterpret_cast<int32_t*>(take(4 * ng));
  d.t_off = reinterpret_cast<int64_t*>(take(8 * (ng + 1)));
  d.s_cnt = reinterpret_cast<int32_t*>(take(4 * ng * kClasses));
  d.s_size = reinterpret_cast<int32_t*>(take(4 * ng));
  d.s_off = reinterpret_cast<int64_t*>(take(8 * (ng + 1)));
  d.s_item_off = reinterpret_cast<int64_t*>(take(8 * (ng + 1)));
  if (w) *w = d;
  return o;
}

// Sizes the workspace layout accepts: non-negative, at most 32 frames per
// group and a table of at most kMaxTable entries (n_groups <= 8192), so every
// byte count of the layout fits in 64 bits.
inline bool derive_sizes_ok(const HierDeriveArgs& a) {
  return a.n_items >= 0 && a.n_groups >= 0 && a.rows >= 0 && a.nq_max >= 0 && a.nq_max <= 32 &&
         (int64_t)a.n_groups * a.n_groups <= kMaxTable;
}

__device__ __forceinline__ void flag(int64_t* totals, int e) {
  atomicOr(reinterpret_cast<unsigned long long*>(&totals[4]), (unsigned long long)e);
}

__global__ void derive_fill_kernel(int32_t* p, int64_t n, int32_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// Up to four fills in one launch (blockIdx.y selects the array).
struct FillJobs {
  int32_t* p[4];
  int64_t n[4];
  int32_t v[4];
};
__global__ void derive_fill4_kernel(FillJobs f) {
  const int j = blockIdx.y;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < f.n[j];
       i += (int64_t)gridDim.x * blockDim.x)
    f.p[j][i] = f.v[j];
}

// Block-wide exclusive scan of one value per thread (kScanThreads threads).
__device__ int64_t block_scan(int64_t v, int64_t* sh, int64_t* total) {
  const int t = threadIdx.x;
  sh[t] = v;
  __syncthreads();
  for (int d = 1; d < kScanThreads; d <<= 1) {
    const int64_t x = t >= d ? sh[t - d] : 0;
    __syncthreads();
    sh[t] += x;
    __syncthreads();
  }
  const int64_t incl = sh[t];
  *total = sh[kScanThreads - 1];
  __syncthreads();
  return incl - v;
}

// Groups: item i starts a group when its row_start is 0; grp_first[n_groups]
// = n_items.  Totals zeroed.
__global__ __launch_bounds__(kScanThreads) void derive_groups_kernel(HierDeriveArgs a, DeriveWs w) {
  __shared__ int64_t sh[kScanThreads];
  const int t = threadIdx.x;
  if (t < 8) a.totals[t] = 0;
  __syncthreads();
  if (t == 0 && (a.n_items < 1 || a.items[3] != 0)) flag(a.totals, kErrItems);
  int64_t carry = 0;
  for (int base = 0; base < a.n_items; base += kScanThreads) {
    const int i = base + t;
    const int32_t* it = a.items + 8 * (int64_t)i;
    const int start = (i < a.n_items && it[3] == 0) ? 1 : 0;
    if (i < a.n_items && (it[7] < 1 || it[7] > a.nq_max || it[2] < 1 || it[5] < 0 ||
                          it[6] < 0 || (int64_t)it[5] + it[6] > a.kv_len))
      flag(a.totals, kErrItems);
    int64_t tot;
    const int64_t ex = block_scan(start, sh, &tot);
    if (i < a.n_items) {
      const int64_t g = carry + ex + start - 1;
      w.grp_of_item[i] = (int32_t)min<int64_t>(max<int64_t>(g, 0), a.n_groups - 1);
      if (start && g < a.n_groups) w.grp_first[g] = i;
    }
    carry += tot;
  }
  if (t == 0) {
    if (carry != a.n_groups) flag(a.totals, kErrItems);
    w.grp_first[a.n_groups] = a.n_items;
  }
}

struct GroupDesc {
  int qbase, qstride, qlen, off, cnt, n;
};

// A group's descriptor, from its first item; the key range is clamped to the
// list (an item outside it is flagged by derive_groups_kernel).
__device__ __forceinline__ GroupDesc group_desc(const HierDeriveArgs& a, const DeriveWs& w, int g) {
  const int32_t* it = a.items + 8 * (int64_t)w.grp_first[g];
  const int off = min(max(it[5], 0), a.kv_len);
  const int cnt = min(max(it[6], 0), a.kv_len - off);
  return {it[0], it[1], max(it[2], 1), off, cnt, it[7]};
}

// token -> (group, row inside the group); items of a group share its list.
__global__ __launch_bounds__(kDeriveThreads) void derive_tokens_kernel(HierDeriveArgs a, DeriveWs w) {
  const int g = blockIdx.x;
  const GroupDesc d = group_desc(a, w, g);
  for (int i = w.grp_first[g] + threadIdx.x; i < w.grp_first[g + 1]; i += blockDim.x) {
    const int32_t* it = a.items + 8 * (int64_t)i;
    if (it[0] != d.qbase || it[1] != d.qstride || it[2] != d.qlen || it[5] != d.off ||
        it[6] != d.cnt || it[7] != d.n)
      flag(a.totals, kErrItems);
  }
  const int nrows = d.n * d.qlen;
  for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
    const int j = r / d.qlen;
    const int64_t tok = (int64_t)d.qbase + (int64_t)j * d.qstride + (r - j * d.qlen);
    if (tok < 0 || tok >= a.rows) {
      flag(a.totals, kErrNoGroup);
      continue;
    }
    if (atomicExch(&w.tok_g[tok], g) != -1) flag(a.totals, kErrTwoGroups);
    w.tok_r[tok] = r;
  }
}

// Runs of query group g's list: every live entry checks that the run of its
// key frame starts where its row says, with the same mask, and is counted
// against its (query group, key group, key frame); each run start checks the
// run's last entry and sets its frame's bit in the key-major table for every
// query frame of its mask.  A complete list has exactly qlen(key group) live
// entries per (g, G, f) that occurs (checked by derive_key_sizes_kernel).
// A group's list is split over gridDim.y workgroups (entries are independent).
__global__ __launch_bounds__(kDeriveThreads) void derive_runs_kernel(HierDeriveArgs a, DeriveWs w) {
  const int g = blockIdx.x;
  const GroupDesc d = group_desc(a, w, g);
  const int ng = a.n_groups, nq = a.nq_max;
  const int lane = threadIdx.x & 63;
  const int32_t* idx = a.kv_idx + d.off;
  const uint32_t* msk = a.kv_mask + d.off;
  for (int i0 = blockIdx.y * kDeriveThreads; i0 < d.cnt; i0 += gridDim.y * kDeriveThreads) {
    const int i = i0 + threadIdx.x;
    int64_t e = -1;                      // counted (g, G, f) of this entry
    const uint32_t m = i < d.cnt ? msk[i] : 0u;
    if (m != 0) {
      const int k = idx[i];
      const int G = (k >= 0 && k < a.rows) ? w.tok_g[k] : -1;
      if (G < 0) {
        flag(a.totals, kErrNoGroup);
      } else {
        const GroupDesc kg = group_desc(a, w, G);
        const int r = w.tok_r[k], f = r / kg.qlen, rin = r - f * kg.qlen;
        const int s = i - rin;
        const int first_tok = kg.qbase + f * kg.qstride;
        if (f < 0 || f >= nq || rin < 0 || s < 0 || idx[s] != first_tok || msk[s] != m) {
          flag(a.totals, kErrRuns);
        } else {
          e = ((int64_t)g * ng + G) * nq + f;
          if (rin == 0) {
            const int last = i + kg.qlen - 1;
            if (last >= d.cnt || idx[last] != first_tok + kg.qlen - 1 || msk[last] != m) {
              flag(a.totals, kErrRuns);
            } else {
              for (int j = 0; j < nq; ++j)
                if ((m >> j) & 1u) atomicOr(&w.table[((int64_t)G * ng + g) * nq + j], 1u << f);
            }
          }
        }
      }
    }
    // one atomic add per distinct run of the wave
    uint64_t rem = __ballot(e >= 0);
    while (rem) {
      const int leader = __ffsll((unsigned long long)rem) - 1;
      const int64_t el = __shfl(e, leader);
      const uint64_t same = __ballot(e == el);
      if (lane == leader) atomicAdd(&w.runs[el], (int)__popcll(same));
      rem &= ~same;
    }
  }
}

// Key-major list size of key group G (padded to 64) and its (query, key) pairs.
__global__ __launch_bounds__(kDeriveThreads) void derive_key_sizes_kernel(HierDeriveArgs a,
                                                                          DeriveWs w) {
  __shared__ int64_t s_size, s_pairs;
  const int G = blockIdx.x;
  const int ng = a.n_groups, nq = a.nq_max;
  if (threadIdx.x == 0) s_size = s_pairs = 0;
  __syncthreads();
  const int qlen_G = group_desc(a, w, G).qlen;
  int64_t size = 0, pairs = 0;
  for (int u = threadIdx.x; u < ng * nq; u += blockDim.x) {
    const int g = u / nq;
    // runs is [query group][key group][key frame]: here query group G, key group g
    const int n_live = w.runs[(int64_t)G * ng * nq + u];
    if (n_live != 0 && n_live != group_desc(a, w, g).qlen) flag(a.totals, kErrRuns);
    const uint32_t bits = w.table[(int64_t)G * ng * nq + u];
    if (bits == 0) continue;
    const int ql = group_desc(a, w, g).qlen;
    size += ql;
    pairs += (int64_t)ql * qlen_G * __popc(bits);
  }
  atomicAdd(reinterpret_cast<unsigned long long*>(&s_size), (unsigned long long)size);
  atomicAdd(reinterpret_cast<unsigned long long*>(&s_pairs), (unsigned long long)pairs);
  __syncthreads();
  if (threadIdx.x == 0) {
    w.t_size[G] = (int32_t)((s_size + kTileKeys - 1) / kTileKeys * kTileKeys);
    atomicAdd(reinterpret_cast<unsigned long long*>(&a.totals[1]), (unsigned long long)s_pairs);
  }
}

// STE selection of one entry (key k, mask m) of the list of the group whose
// query rows start at token qbase: class, or -1 if not kept.
__device__ __forceinline__ int ste_class_at(const HierDeriveArgs& a, int64_t qbase, int k,
                                            uint32_t m) {
  const int64_t a0 = (int64_t)a.P * a.T * a.L, g0 = a0 + (int64_t)a.T * a.N * a.KL;
  if (m == 0 || k < 0 || qbase >= g0) return -1;
  if (qbase < a0) {
    if (k < a0 || k >= g0) return -1;
    return (int)(((k - a0) / max(a.KL, 1)) % max(a.N, 1));
  }
  if (k >= a0) return -1;
  return (int)(k / ((int64_t)a.T * a.L));
}

__device__ __forceinline__ int ste_class(const HierDeriveArgs& a, const GroupDesc& d, int k,
                                         uint32_t m) {
  return ste_class_at(a, d.qbase, k, m);
}

// Class of every entry of item i's list, written by every item over its own
// range (the items of a group write the same values; a cut item covers part
// of its group's list; entries outside [0, kv_len) are never written), and
// the first 64-entry tile of the item's range holding a class.
__global__ __launch_bounds__(kDeriveThreads) void derive_fwd_class_kernel(HierDeriveArgs a,
                                                                         int32_t* cls,
                                                                         int32_t* first) {
  __shared__ int s_first;
  const int32_t* it = a.items + 8 * (int64_t)blockIdx.x;
  const int64_t qbase = it[0], off = it[5], cnt = it[6];
  if (threadIdx.x == 0) s_first = INT_MAX;
  __syncthreads();
  const int64_t lo = max(off, (int64_t)0), hi = min(off + cnt, (int64_t)a.kv_len);
  int mine = INT_MAX;   // this thread's first entry with a class (its entries ascend)
  for (int64_t e = lo + threadIdx.x; e < hi; e += blockDim.x) {
    const int c = ste_class_at(a, qbase, a.kv_idx[e], a.kv_mask[e]);
    cls[e] = c;
    if (c >= 0 && mine == INT_MAX) mine = (int)(e - off);
  }
  if (mine != INT_MAX) atomicMin(&s_first, mine);
  __syncthreads();
  if (threadIdx.x == 0)
    first[blockIdx.x] = s_first == INT_MAX ? (int)((max(cnt, (int64_t)0) + kTileKeys - 1) / kTileKeys)
                                           : s_first / kTileKeys;
}

__device__ __forceinline__ bool ste_group(const HierDeriveArgs& a, const GroupDesc& d) {
  const int64_t a0 = (int64_t)a.P * a.T * a.L, g0 = a0 + (int64_t)a.T * a.N * a.KL;
  return d.qbase < g0 && d.cnt > 0;
}

// Per-class counts of group g's STE list.
__global__ __launch_bounds__(kDeriveThreads) void derive_ste_count_kernel(HierDeriveArgs a,
                                                                         DeriveWs w) {
  __shared__ int cnt[kClasses];
  const int g = blockIdx.x;
  for (int c = threadIdx.x; c < kClasses; c += blockDim.x) cnt[c] = 0;
  __syncthreads();
  const GroupDesc d = group_desc(a, w, g);
  if (ste_group(a, d))
    for (int i = threadIdx.x; i < d.cnt; i += blockDim.x) {
      const int c = ste_class(a, d, a.kv_idx[d.off + i], a.kv_mask[d.off + i]);
      if (c >= kClasses) flag(a.totals, kErrItems);
      else if (c >= 0) atomicAdd(&cnt[c], 1);
    }
  __syncthreads();
  int n = 0;
  for (int c = 0; c < kClasses; ++c) n += cnt[c];
  for (int c = threadIdx.x; c < kClasses; c += blockDim.x) w.s_cnt[g * kClasses + c] = cnt[c];
  if (threadIdx.x == 0) w.s_size[g] = (n + kTileKeys - 1) / kTileKeys * kTileKeys;
}

// Offsets of both lists and of the STE items; totals [0] key-major entries,
// [2] STE entries, [3] STE items.
__global__ __launch_bounds__(kScanThreads) void derive_scan_kernel(HierDeriveArgs a, DeriveWs w) {
  __shared__ int64_t sh[kScanThreads];
  int64_t ct = 0, cs = 0, ci = 0;
  for (int base = 0; base < a.n_groups; base += kScanThreads) {
    const int g = base + threadIdx.x;
    const bool in = g < a.n_groups;
    const int64_t vt = in ? w.t_size[g] : 0, vs = in ? w.s_size[g] : 0;
    const int64_t vi = (in && vs > 0) ? (int64_t)(w.grp_first[g + 1] - w.grp_first[g]) : 0;
    int64_t tt, ts, ti;
    const int64_t et = block_scan(vt, sh, &tt);
    const int64_t es = block_scan(vs, sh, &ts);
    const int64_t ei = block_scan(vi, sh, &ti);
    if (in) {
      w.t_off[g] = ct + et;
      w.s_off[g] = cs + es;
      w.s_item_off[g] = ci + ei;
    }
    ct += tt;
    cs += ts;
    ci += ti;
  }
  if (threadIdx.x == 0) {
    w.t_off[a.n_groups] = ct;
    w.s_off[a.n_groups] = cs;
    w.s_item_off[a.n_groups] = ci;
    a.totals[0] = ct;
    a.totals[2] = cs;
    a.totals[3] = ci;
    if (ct > INT32_MAX || cs > INT32_MAX) flag(a.totals, kErrOverflow);
  }
}

// Key-major list of key group G: unit offsets by a block scan over the
// (g, j) units, then every entry finds its unit by binary search.
__global__ __launch_bounds__(kScanThreads) void derive_key_write_kernel(HierDeriveArgs a,
                                                                        DeriveWs w) {
  __shared__ int64_t sh[kScanThreads];
  __shared__ int32_t u_off[kScanThreads];
  __shared__ int32_t u_id[kScanThreads];
  // after a flagged pass 1 the offsets are not trusted: nothing is written
  if (a.totals[4] != 0) return;
  const int G = blockIdx.x;
  const int ng = a.n_groups, nq = a.nq_max, nu = ng * nq;
  const int64_t base = w.t_off[G];
  const int64_t lim = a.key_entries;   // the caller's list size bounds every store
  const int padded = w.t_size[G];
  const uint32_t* row = w.table + (int64_t)G * nu;
  int64_t done = 0;   // entries written before this chunk of units
  for (int u0 = 0; u0 < nu; u0 += kScanThreads) {
    const int u = u0 + threadIdx.x;
    const int g = u / nq;
    const bool live = u < nu && row[u] != 0;
    const int len = live ? group_desc(a, w, g).qlen : 0;
    int64_t chunk, n_live;
    const int64_t ex = block_scan(len, sh, &chunk);
    // the live units of this chunk, compacted in order
    const int64_t li = block_scan(live ? 1 : 0, sh, &n_live);
    if (live) {
      u_off[li] = (int32_t)ex;
      u_id[li] = u;
    }
    __syncthreads();
    const int nl = (int)n_live;
    for (int p = threadIdx.x; p < chunk; p += blockDim.x) {
      int lo = 0, hi = nl - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (u_off[mid] <= p) lo = mid; else hi = mid - 1;
      }
      const int uu = u_id[lo], gg = uu / nq, j = uu - gg * nq;
      const GroupDesc q = group_desc(a, w, gg);
      const int r = p - u_off[lo];
      const int64_t o = base + done + p;
      if (o < lim) {
        a.key_q_idx[o] = q.qbase + j * q.qstride + r;
        a.key_q_mask[o] = row[uu];
      }
    }
    done += chunk;
    __syncthreads();
  }
  for (int64_t p = done + threadIdx.x; p < padded && base + p < lim; p += blockDim.x) {
    a.key_q_idx[base + p] = 0;
    a.key_q_mask[base + p] = 0;
  }
}

// STE list of group g: entries in list order, stably grouped by class.  Each
// chunk of 256 entries ranks its entries per class with wave ballots; a
// running count per class carries the order across chunks.
__global__ __launch_bounds__(kDeriveThreads) void derive_ste_write_kernel(HierDeriveArgs a,
                                                                         DeriveWs w) {
  __shared__ int cbase[kClasses];     // first position of each class in the list
  __shared__ int wcnt[kDeriveThreads / 64][kClasses];
  if (a.totals[4] != 0) return;       // flagged pass 1: nothing is written
  const int g = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const GroupDesc d = group_desc(a, w, g);
  const int padded = w.s_size[g];
  if (padded == 0) return;
  const int64_t base = w.s_off[g];
  const int64_t lim = a.ste_entries, item_lim = a.totals[3];
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int c = 0; c < kClasses; ++c) {
      cbase[c] = acc;
      acc += w.s_cnt[g * kClasses + c];
    }
  }
  __syncthreads();
  for (int i0 = 0; i0 < d.cnt; i0 += kDeriveThreads) {
    const int i = i0 + threadIdx.x;
    int k = 0, c = -1;
    uint32_t m = 0;
    if (i < d.cnt) {
      k = a.kv_idx[d.off + i];
      m = a.kv_mask[d.off + i];
      c = ste_class(a, d, k, m);
      if (c >= kClasses) c = -1;
    }
    for (int cc = lane; cc < kClasses; cc += 64) wcnt[wave][cc] = 0;
    // rank inside the wave: one ballot per distinct class present
    int rank = 0;
    uint64_t rem = __ballot(c >= 0);
    while (rem) {
      const int leader = __ffsll((unsigned long long)rem) - 1;
      const int cl = __shfl(c, leader);
      const uint64_t same = __ballot(c == cl);
      if (c == cl) rank = __popcll(same & ((1ull << lane) - 1));
      if (lane == 0) wcnt[wave][cl] = __popcll(same);
      rem &= ~same;
    }
    __syncthreads();
    if (c >= 0) {
      int before = 0;
      for (int v = 0; v < wave; ++v) before += wcnt[v][c];
      const int64_t pos = base + cbase[c] + before + rank;
      if (pos < lim) {
        a.ste_kv_idx[pos] = k;
        a.ste_kv_mask[pos] = m;
        a.ste_kv_class[pos] = c;
      }
    }
    __syncthreads();
    for (int cc = threadIdx.x; cc < kClasses; cc += blockDim.x) {
      int n = 0;
      for (int v = 0; v < kDeriveThreads / 64; ++v) n += wcnt[v][cc];
      cbase[cc] += n;
    }
    __syncthreads();
  }
  int n = 0;
  for (int c = 0; c < kClasses; ++c) n += w.s_cnt[g * kClasses + c];
  for (int p = n + threadIdx.x; p < padded && base + p < lim; p += blockDim.x) {
    a.ste_kv_idx[base + p] = 0;
    a.ste_kv_mask[base + p] = 0;
    a.ste_kv_class[base + p] = 0;
  }
  // the group's STE items
  const int first = w.grp_first[g], end = w.grp_first[g + 1];
  for (int i = first + threadIdx.x; i < end; i += blockDim.x) {
    const int64_t o = w.s_item_off[g] + (i - first);
    if (o >= item_lim) break;
    for (int e = 0; e < 8; ++e) a.ste_items[8 * o + e] = a.items[8 * (int64_t)i + e];
    a.ste_items[8 * o + 5] = (int32_t)base;
    a.ste_items[8 * o + 6] = base + padded <= lim ? padded : 0;
  }
}

// Key-major items: the forward items with their group's list offset / size.
__global__ void derive_key_items_kernel(HierDeriveArgs a, DeriveWs w) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.n_items) return;
  for (int e = 0; e < 8; ++e) a.key_items[8 * (int64_t)i + e] = a.items[8 * (int64_t)i + e];
  // a flagged pass 1 or a list past the caller's size: an empty list (the
  // backward then reads nothing through this item)
  const bool ok = a.totals[4] == 0;
  const int g = ok ? w.grp_of_item[i] : 0;
  const bool fits = ok && w.t_off[g] + w.t_size[g] <= a.key_entries;
  a.key_items[8 * (int64_t)i + 5] = fits ? (int32_t)w.t_off[g] : 0;
  a.key_items[8 * (int64_t)i + 6] = fits ? w.t_size[g] : 0;
}

// AND of the masks of every 64 entries (one wave per tile).
__global__ void derive_blk_and_kernel(const uint32_t* mask, uint32_t* blk, int64_t n_tiles) {
  const int64_t tile = blockIdx.x * (int64_t)(blockDim.x / 64) + (threadIdx.x >> 6);
  if (tile >= n_tiles) return;
  uint32_t v = mask[tile * 64 + (threadIdx.x & 63)];
  for (int s = 32; s >= 1; s >>= 1) v &= __shfl_xor(v, s);
  if ((threadIdx.x & 63) == 0) blk[tile] = v;
}

int derive_validate(const HierDeriveArgs* a, DeriveWs* w) {
  HIER_REQUIRE(a != nullptr, HIER_EINVAL, "args is NULL");
  HIER_REQUIRE(a->n_items >= 1 && a->n_groups >= 1 && a->rows >= 1 && a->nq_max >= 1 &&
                   a->nq_max <= 32,
               HIER_EINVAL, "invalid n_items=%d n_groups=%d rows=%d nq_max=%d", a->n_items,
               a->n_groups, a->rows, a->nq_max);
  HIER_REQUIRE((int64_t)a->n_groups * a->n_groups <= kMaxTable / a->nq_max, HIER_EUNSUPPORTED,
               "too many groups for the device transposer (%d groups x %d frames)", a->n_groups,
               a->nq_max);
  HIER_REQUIRE(a->kv_len >= 0, HIER_EINVAL, "invalid kv_len=%d", a->kv_len);
  HIER_REQUIRE(a->P >= 0 && a->T >= 0 && a->L >= 0 && a->N >= 0 && a->KL >= 0, HIER_EINVAL,
               "invalid STE geometry");
  HIER_REQUIRE(a->items && a->kv_idx && a->kv_mask && a->totals && a->ws, HIER_EINVAL,
               "NULL input pointer");
  const int64_t need = derive_ws_layout(*a, w);
  HIER_REQUIRE(a->ws_bytes >= need, HIER_EINVAL, "workspace holds %lld bytes, %lld needed",
               (long long)a->ws_bytes, (long long)need);
  return HIER_OK;
}

void fill(int32_t* p, int64_t n, int32_t v, hipStream_t s) {
  const int grid = (int)std::min<int64_t>((n + 255) / 256, 4096);
  if (grid > 0) hipLaunchKernelGGL(derive_fill_kernel, dim3(grid), dim3(256), 0, s, p, n, v);
}

}  // namespace

extern "C" int64_t hier_derive_workspace(const HierDeriveArgs* args) {
  if (!args || !derive_sizes_ok(*args)) return -1;
  HierDeriveArgs a = *args;
  a.ws = nullptr;
  return derive_ws_layout(a, nullptr);
}

extern "C" int hier_derive_count(const HierDeriveArgs* args, void* stream) {
  hier::clear_error();
  DeriveWs w;
  int rc = derive_validate(args, &w);
  if (rc) return rc;
  const HierDeriveArgs& a = *args;
  hipStream_t s = (hipStream_t)stream;
  const int64_t tab = (int64_t)a.n_groups * a.n_groups * a.nq_max;
  FillJobs fj = {{w.grp_first, w.tok_g, reinterpret_cast<int32_t*>(w.table), w.runs},
                 {(int64_t)a.n_groups + 1, a.rows, tab, tab},
                 {0, -1, 0, 0}};
  const int64_t fmax = std::max<int64_t>(std::max<int64_t>(a.n_groups + 1, a.rows), tab);
  hipLaunchKernelGGL(derive_fill4_kernel, dim3((unsigned)std::min<int64_t>((fmax + 255) / 256, 1024), 4),
                     dim3(256), 0, s, fj);
  hipLaunchKernelGGL(derive_groups_kernel, dim3(1), dim3(kScanThreads), 0, s, a, w);
  hipLaunchKernelGGL(derive_tokens_kernel, dim3(a.n_groups), dim3(kDeriveThreads), 0, s, a, w);
  hipLaunchKernelGGL(derive_runs_kernel, dim3(a.n_groups, kRunSplit), dim3(kDeriveThreads), 0, s,
                     a, w);
  hipLaunchKernelGGL(derive_key_sizes_kernel, dim3(a.n_groups), dim3(kDeriveThreads), 0, s, a, w);
  hipLaunchKernelGGL(derive_ste_count_kernel, dim3(a.n_groups), dim3(kDeriveThreads), 0, s, a, w);
  hipLaunchKernelGGL(derive_scan_kernel, dim3(1), dim3(kScanThreads), 0, s, a, w);
  return hier::check_launch("derive count kernels");
}

extern "C" int hier_derive_ste_classes(const HierDeriveArgs* args, int32_t* kv_class,
                                       int32_t* item_first, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr && kv_class != nullptr && item_first != nullptr, HIER_EINVAL,
               "NULL args, kv_class or item_first");
  const HierDeriveArgs& a = *args;
  HIER_REQUIRE(a.n_items >= 0 && a.kv_len >= 0, HIER_EINVAL, "invalid n_items=%d kv_len=%d",
               a.n_items, a.kv_len);
  HIER_REQUIRE(a.P >= 0 && a.T >= 0 && a.L >= 0 && a.N >= 0 && a.KL >= 0, HIER_EINVAL,
               "invalid STE geometry");
  HIER_REQUIRE(a.n_items == 0 || (a.items && a.kv_idx && a.kv_mask), HIER_EINVAL,
               "NULL input pointer");
  hipStream_t s = (hipStream_t)stream;
  fill(kv_class, a.kv_len, -1, s);
  if (a.n_items > 0)
    hipLaunchKernelGGL(derive_fwd_class_kernel, dim3(a.n_items), dim3(kDeriveThreads), 0, s, a,
                       kv_class, item_first);
  return hier::check_launch("derive_fwd_class_kernel");
}

extern "C" int hier_derive_build(const HierDeriveArgs* args, void* stream) {
  hier::clear_error();
  DeriveWs w;
  int rc = derive_validate(args, &w);
  if (rc) return rc;
  const HierDeriveArgs& a = *args;
  HIER_REQUIRE(a.key_items && a.key_q_idx && a.key_q_mask && a.key_blk_and, HIER_EINVAL,
               "key-major output pointer is NULL");
  HIER_REQUIRE(a.key_entries >= 0 && a.key_entries % kTileKeys == 0 && a.ste_entries >= 0 &&
                   a.ste_entries % kTileKeys == 0,
               HIER_EINVAL, "list sizes must be the multiples of 64 that pass 1 returned");
  const bool ste = a.ste_entries > 0;
  if (ste)
    HIER_REQUIRE(a.ste_items && a.ste_kv_idx && a.ste_kv_mask && a.ste_blk_and && a.ste_kv_class,
                 HIER_EINVAL, "STE output pointer is NULL");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(derive_key_write_kernel, dim3(a.n_groups), dim3(kScanThreads), 0, s, a, w);
  hipLaunchKernelGGL(derive_key_items_kernel, dim3((a.n_items + 255) / 256), dim3(256), 0, s, a,
                     w);
  const int64_t kt = a.key_entries / kTileKeys;
  if (kt > 0)
    hipLaunchKernelGGL(derive_blk_and_kernel, dim3((unsigned)((kt + 3) / 4)), dim3(256), 0, s,
                       a.key_q_mask, a.key_blk_and, kt);
  if (ste) {
    hipLaunchKernelGGL(derive_ste_write_kernel, dim3(a.n_groups), dim3(kDeriveThreads), 0, s, a,
                       w);
    const int64_t st = a.ste_entries / kTileKeys;
    hipLaunchKernelGGL(derive_blk_and_kernel, dim3((unsigned)((st + 3) / 4)), dim3(256), 0, s,
                       a.ste_kv_mask, a.ste_blk_and, st);
  }
  return hier::check_launch("derive build kernels");
}

// ---- membership-dependent topology arrays from soft logits -----------------
//
// membership = logits > 0; global_only[t][p] = p in no group at t;
// q_active[b][j][g] = group g has a member at frame b*n + j;
// local_active[b][g][fi] = group g has a member at frame la_frame[b][fi]
// (0 for a padding column, la_frame < 0).  The arrays a membership topology
// derives from its membership (hier_masks.py:127-193), one launch.
namespace {

__device__ __forceinline__ bool any_member(const HierMembershipArgs& a, int t, int g) {
  const float* l = a.logits + ((int64_t)t * a.N + g) * a.P;
  bool any = false;
  for (int p = 0; p < a.P; ++p) any |= l[p] > 0.f;
  return any;
}

__global__ __launch_bounds__(256) void membership_kernel(HierMembershipArgs a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n_mem = (int64_t)a.T * a.N * a.P, n_go = (int64_t)a.T * a.P;
  const int64_t n_qa = (int64_t)a.B * a.n * a.N, n_la = (int64_t)a.B * a.N * a.fl_max;
  if (i < n_mem) a.membership[i] = a.logits[i] > 0.f ? 1 : 0;
  if (i < n_go) {
    const int t = (int)(i / a.P), p = (int)(i % a.P);
    bool in = false;
    for (int g = 0; g < a.N; ++g) in |= a.logits[((int64_t)t * a.N + g) * a.P + p] > 0.f;
    a.global_only[i] = in ? 0 : 1;
  }
  if (i < n_qa) {
    const int g = (int)(i % a.N);
    const int64_t bj = i / a.N;                       // b * n + j = the frame
    a.q_active[i] = any_member(a, (int)bj, g) ? 1 : 0;
  }
  if (i < n_la) {
    const int fi = (int)(i % a.fl_max);
    const int64_t bg = i / a.fl_max;
    const int g = (int)(bg % a.N), b = (int)(bg / a.N);
    const int f = a.la_frame[(int64_t)b * a.fl_max + fi];
    a.local_active[i] = (f >= 0 && f < a.T && any_member(a, f, g)) ? 1 : 0;
  }
}

}  // namespace

extern "C" int hier_membership_from_logits(const HierMembershipArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  const HierMembershipArgs& a = *args;
  HIER_REQUIRE(a.T >= 1 && a.N >= 1 && a.P >= 1 && a.B >= 1 && a.n >= 1 && a.fl_max >= 0 &&
                   a.T <= (1 << 20) && a.N <= 1024 && a.P <= 1024 && a.fl_max <= (1 << 20) &&
                   (int64_t)a.B * a.n == a.T,
               HIER_EINVAL, "invalid T=%d N=%d P=%d B=%d n=%d fl_max=%d", a.T, a.N, a.P, a.B, a.n,
               a.fl_max);
  HIER_REQUIRE(a.logits && a.membership && a.global_only && a.q_active &&
                   (a.fl_max == 0 || (a.la_frame && a.local_active)),
               HIER_EINVAL, "NULL pointer");
  const int64_t n = std::max<int64_t>((int64_t)a.T * a.N * a.P, (int64_t)a.B * a.N * a.fl_max);
  hipLaunchKernelGGL(membership_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, a);
  return hier::check_launch("membership_kernel");
}

// ---- hub streams merged across temporal blocks -----------------------------
//
// A local-hub slot or the global hub has few query rows per block (n * KL,
// n * KG) but a long key list, so one work item per (block, hub stream)
// streams a whole list for one wave of rows.  The rows of G consecutive blocks
// of one hub stream form one group instead: its list is the union of the G
// source lists (each a concatenation of whole key frames), a key's mask bits
// of block b0 + j shifted by n * j (bit f = the group's query frame f).  Pass
// A scatters every live source entry into a dense per-group mask array over
// the key rows (atomic OR); pass B compacts each group's array in row order
// into the group's slot (its capacity, the sum of its sources' sizes, bounds
// the union), pads it to 64 with mask 0, writes the per-64 mask ANDs and the
// group's work items.  Key frames stay contiguous in row order, as the
// backward's derivation requires.
//
// A forward-only group may also take the ragged last item of the players
// that belong to its hub: that item has a few rows (n * L mod 128) but walks
// the player's whole list, and a member's keys are a subset of its hub's, so
// its rows join the hub's items at no extra key.  Such a source contributes
// only the bits of its rows' query frames (src_from / src_nbits), shifted to
// bits of their own; the group's items then read their (token, bit) rows
// from a row table.
namespace {

constexpr int kMergeThreads = 1024;

__global__ __launch_bounds__(256) void merge_scatter_kernel(HierMergeArgs a) {
  const int i = blockIdx.x;                              // source list
  const int32_t* it = a.items + 8 * (int64_t)a.src_item[i];
  const int64_t off = it[5];
  const int cnt = it[6];
  const int g = a.src_group[i], sh = a.src_shift[i];
  int from = 0;
  uint32_t keep = ~0u;
  if (a.src_from != nullptr) {
    from = a.src_from[i] & 31;
    const int nb = a.src_nbits[i];
    keep = nb >= 32 ? ~0u : (nb <= 0 ? 0u : (1u << nb) - 1u);
  }
  uint32_t* acc = a.acc + (int64_t)g * a.rows;
  for (int e = blockIdx.y * blockDim.x + threadIdx.x; e < cnt; e += gridDim.y * blockDim.x) {
    const uint32_t m = (a.kv_mask[off + e] >> from) & keep;
    const int k = a.kv_idx[off + e];
    if (m != 0 && k >= 0 && k < a.rows) atomicOr(&acc[k], m << sh);
  }
}

__global__ __launch_bounds__(kMergeThreads) void merge_compact_kernel(HierMergeArgs a) {
  __shared__ int wsum[kMergeThreads / 64];
  __shared__ int base_s, first_s;
  const int g = blockIdx.x;
  const uint32_t* acc = a.acc + (int64_t)g * a.rows;
  const int64_t out = a.out_off[g];
  const int cap = a.out_cap[g];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) {
    base_s = 0;
    first_s = -1;
  }
  __syncthreads();
  // four consecutive rows per thread and pass, in row order: a thread's live
  // rows follow those of the lower lanes of its wave and of the lower waves
  constexpr int kRows = 4 * kMergeThreads;
  for (int r0 = 0; r0 < a.rows; r0 += kRows) {
    const int rb = r0 + 4 * threadIdx.x;
    uint32_t m[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) m[e] = rb + e < a.rows ? acc[rb + e] : 0u;
    const int mine = (m[0] != 0) + (m[1] != 0) + (m[2] != 0) + (m[3] != 0);
    int incl = mine;                       // inclusive prefix over the wave's lanes
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d, 64);
      if (lane >= d) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int before = 0, total = 0;
    for (int w = 0; w < kMergeThreads / 64; ++w) {
      before += w < wave ? wsum[w] : 0;
      total += wsum[w];
    }
    int pos = base_s + before + incl - mine;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (m[e] == 0) continue;
      if (pos < cap) {
        a.kv_idx[out + pos] = rb + e;
        a.kv_mask[out + pos] = m[e];
      }
      if (pos == 0) first_s = rb + e;
      ++pos;
    }
    __syncthreads();
    if (threadIdx.x == 0) base_s += total;
    __syncthreads();
  }
  const int uni = min(base_s, cap);
  const int padded = min((uni + 63) / 64 * 64, cap);
  const int pad_idx = first_s < 0 ? 0 : first_s;
  for (int p = uni + threadIdx.x; p < padded; p += blockDim.x) {
    a.kv_idx[out + p] = pad_idx;
    a.kv_mask[out + p] = 0;
  }
  __syncthreads();
  for (int t = threadIdx.x; t < padded / 64; t += blockDim.x) {
    uint32_t x = ~0u;
    for (int e = 0; e < 64; ++e) x &= a.kv_mask[out + 64 * t + e];
    a.blk_and[out / 64 + t] = x;
  }
  // the group's items: rows split into rows_per_item pieces
  const int32_t* d = a.group_desc + 4 * (int64_t)g;      // qbase, qstride, qlen, frames
  const int rows = d[2] * d[3];
  const int nit = (rows + a.rows_per_item - 1) / a.rows_per_item;
  for (int it = threadIdx.x; it < nit; it += blockDim.x) {
    int32_t* o = a.out_items + 8 * ((int64_t)a.group_item_off[g] + it);
    o[0] = d[0];
    o[1] = d[1];
    o[2] = d[2];
    o[3] = it * a.rows_per_item;
    o[4] = min(a.rows_per_item, rows - it * a.rows_per_item);
    o[5] = (int32_t)out;
    o[6] = padded;
    o[7] = d[3];
  }
}

}  // namespace

extern "C" int hier_merge_hub_lists(const HierMergeArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  const HierMergeArgs& a = *args;
  HIER_REQUIRE(a.n_groups >= 0 && a.n_src >= 0 && a.rows >= 1 && a.rows_per_item >= 32 &&
                   a.rows_per_item % 32 == 0 && (int64_t)a.n_groups * a.rows <= (1ll << 31),
               HIER_EINVAL, "invalid n_groups=%d n_src=%d rows=%d rows_per_item=%d", a.n_groups,
               a.n_src, a.rows, a.rows_per_item);
  if (a.n_groups == 0) return HIER_OK;
  HIER_REQUIRE(a.items && a.kv_idx && a.kv_mask && a.blk_and && a.acc && a.src_item &&
                   a.src_group && a.src_shift && a.out_off && a.out_cap && a.group_desc &&
                   a.group_item_off && a.out_items,
               HIER_EINVAL, "NULL pointer");
  HIER_REQUIRE((a.src_from == nullptr) == (a.src_nbits == nullptr), HIER_EINVAL,
               "src_from and src_nbits must both be set or both be NULL");
  hipStream_t s = (hipStream_t)stream;
  const int64_t n_acc = (int64_t)a.n_groups * a.rows;
  hipLaunchKernelGGL(derive_fill_kernel, dim3((unsigned)std::min<int64_t>((n_acc + 255) / 256, 4096)),
                     dim3(256), 0, s, reinterpret_cast<int32_t*>(a.acc), n_acc, 0);
  if (a.n_src > 0)
    hipLaunchKernelGGL(merge_scatter_kernel, dim3(a.n_src, 4), dim3(256), 0, s, a);
  hipLaunchKernelGGL(merge_compact_kernel, dim3(a.n_groups), dim3(kMergeThreads), 0, s, a);
  return hier::check_launch("merge kernels");
}

// ---- key lists cut to the tiles their rows see ------------------------------
//
// One workgroup per item: the OR of its rows' mask bits, then the first and
// last 64-entry tile holding an entry with one of those bits (each thread's
// own minimum / maximum, then one LDS atomic per thread).  The item's words
// are read into LDS before any is written, so the output may alias the input.
namespace {

constexpr int kTrimThreads = 256;

__global__ __launch_bounds__(kTrimThreads) void trim_kernel(HierTrimArgs a) {
  __shared__ int32_t it[8];
  __shared__ uint32_t bits_s;
  __shared__ int first_s, last_s;
  const int64_t i = blockIdx.x;
  if (threadIdx.x < 8) it[threadIdx.x] = a.items[8 * i + threadIdx.x];
  if (threadIdx.x == 0) {
    bits_s = 0u;
    first_s = INT_MAX;
    last_s = -1;
  }
  __syncthreads();
  const int qbase = it[0], qstride = it[1], qlen = it[2], r0 = it[3], rc = it[4];
  const int64_t off = it[5];
  const int cnt = it[6];
  uint32_t bits = 0u;
  for (int r = threadIdx.x; r < rc; r += blockDim.x) {
    int bit = -1;
    if (qstride < 0) {
      if (a.row_table != nullptr) bit = a.row_table[2 * ((int64_t)qbase + r0 + r) + 1];
    } else if (qlen > 0) {
      bit = (r0 + r) / qlen;
    }
    if (bit >= 0 && bit < 32) bits |= 1u << bit;
  }
  if (bits != 0u) atomicOr(&bits_s, bits);
  __syncthreads();
  bits = bits_s;
  int lo = INT_MAX, hi = -1;
  // four entries per load where the range allows (lists start on 64-entry
  // tiles, so off is a multiple of 4 for every list this library builds)
  const int n4 = (off & 3) == 0 ? cnt >> 2 : 0;
  const uint4* m4 = reinterpret_cast<const uint4*>(a.kv_mask + off);
  for (int q = threadIdx.x; q < n4; q += blockDim.x) {
    const uint4 w = m4[q];
    const bool any = ((w.x | w.y | w.z | w.w) & bits) != 0u;
    if (any) {
      lo = min(lo, q >> 4);
      hi = max(hi, q >> 4);
    }
  }
  for (int e = 4 * n4 + threadIdx.x; e < cnt; e += blockDim.x)
    if (a.kv_mask[off + e] & bits) {
      lo = min(lo, e >> 6);
      hi = max(hi, e >> 6);
    }
  if (hi >= 0) {
    atomicMin(&first_s, lo);
    atomicMax(&last_s, hi);
  }
  __syncthreads();
  if (threadIdx.x < 8) {
    int32_t v = it[threadIdx.x];
    if (last_s >= 0 && threadIdx.x == 5) v = (int32_t)(off + 64 * (int64_t)first_s);
    if (last_s >= 0 && threadIdx.x == 6) v = min(cnt - 64 * first_s, 64 * (last_s - first_s + 1));
    a.out_items[8 * i + threadIdx.x] = v;
  }
}

}  // namespace

extern "C" int hier_trim_key_lists(const HierTrimArgs* args, void* stream) {
  hier::clear_error();
  HIER_REQUIRE(args != nullptr, HIER_EINVAL, "args is NULL");
  const HierTrimArgs& a = *args;
  HIER_REQUIRE(a.n_items >= 0, HIER_EINVAL, "invalid n_items=%d", a.n_items);
  if (a.n_items == 0) return HIER_OK;
  HIER_REQUIRE(a.items && a.kv_mask && a.out_items, HIER_EINVAL, "NULL pointer");
  hipLaunchKernelGGL(trim_kernel, dim3(a.n_items), dim3(kTrimThreads), 0, (hipStream_t)stream, a);
  return hier::check_launch("trim_kernel");
}
