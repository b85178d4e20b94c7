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
