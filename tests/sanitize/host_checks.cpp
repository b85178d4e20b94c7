// Host-side checks of the C ABI under AddressSanitizer and
// UndefinedBehaviorSanitizer (host code only; no GPU, no kernel launch).
//
// Every call below either fails an argument check -- the expected HIER_E*
// code and a non-empty hier_last_error() -- or returns before its first
// launch (empty work), so the library's host paths run with hostile and
// extreme values: NULL and misaligned pointers, negative and huge sizes and
// strides, sizes whose products overflow 64 bits.  Device pointers are
// stand-in addresses that host code must never dereference (ASan reports a
// host read of one).  The derive workspace sizing is evaluated over a grid
// of sizes, its monotonicity checked.  Exit status = number of failed checks.
#include <climits>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "hierattn.h"

static int g_fail = 0;

static void expect(int rc, int want, const char* what, int line) {
  const char* msg = hier_last_error();
  if (rc != want) {
    std::printf("FAIL line %d %s: rc %d, expected %d (%s)\n", line, what, rc, want, msg);
    ++g_fail;
  } else if (want != HIER_OK && (msg == nullptr || msg[0] == 0)) {
    std::printf("FAIL line %d %s: no error message\n", line, what);
    ++g_fail;
  } else if (want == HIER_OK && msg[0] != 0) {
    std::printf("FAIL line %d %s: message %s after success\n", line, what, msg);
    ++g_fail;
  }
}
#define EXPECT(call, want) expect((call), (want), #call, __LINE__)

// Stand-in device addresses: 16-byte aligned, never dereferenced on the host.
template <class T>
static T* dev(uintptr_t slot) {
  return reinterpret_cast<T*>((uintptr_t)0x7f0000000000ull + slot * 0x100000ull);
}

static HierTopo good_topo() {
  HierTopo t;
  std::memset(&t, 0, sizeof(t));
  t.P = 4; t.N = 2; t.L = 220; t.KL = 5; t.KG = 6; t.n_frames = 3; t.n_block = 3;
  t.local_attn = 21; t.direct = 1; t.B = 14; t.fa_max = 24; t.fl_max = 24; t.fg_max = 24;
  t.fa = dev<int32_t>(1); t.fl = dev<int32_t>(2); t.fg = dev<int32_t>(3);
  t.agent_frames = dev<int32_t>(4); t.local_frames = dev<int32_t>(5);
  t.global_frames = dev<int32_t>(6); t.local_active = dev<uint8_t>(7);
  t.q_frames = dev<int32_t>(8); t.labels = dev<int32_t>(9); t.q_active = dev<uint8_t>(10);
  t.ref_agent_base = dev<int32_t>(11); t.ref_local_base = dev<int32_t>(12);
  t.ref_global_base = dev<int32_t>(13); t.tile_agent_base = dev<int32_t>(14);
  t.tile_local_base = dev<int32_t>(15); t.tile_global_base = dev<int32_t>(16);
  t.ref_qbase = dev<int32_t>(17); t.tile_qbase = dev<int32_t>(18);
  return t;
}

static void meta_checks() {
  EXPECT(hier_meta_count(nullptr, nullptr, nullptr), HIER_EINVAL);
  HierTopo t = good_topo();
  EXPECT(hier_meta_count(&t, nullptr, nullptr), HIER_EINVAL);      // counts missing
  EXPECT(hier_meta_build(&t, nullptr, nullptr), HIER_EINVAL);      // output missing
  HierMetaOut out;
  std::memset(&out, 0, sizeof(out));
  out.tile_kv_idx = dev<int32_t>(20);                              // tile list half given
  EXPECT(hier_meta_build(&t, &out, nullptr), HIER_EINVAL);
  struct Bad { int HierTopo::*f; int v; int want; } bad[] = {
      {&HierTopo::P, 0, HIER_EINVAL},          {&HierTopo::P, INT_MAX, HIER_EUNSUPPORTED},
      {&HierTopo::N, INT_MAX, HIER_EUNSUPPORTED}, {&HierTopo::L, -1, HIER_EINVAL},
      {&HierTopo::L, INT_MAX, HIER_EUNSUPPORTED}, {&HierTopo::KL, -5, HIER_EINVAL},
      {&HierTopo::n_frames, 0, HIER_EUNSUPPORTED}, {&HierTopo::n_frames, 33, HIER_EUNSUPPORTED},
      {&HierTopo::n_block, 0, HIER_EINVAL},    {&HierTopo::B, 0, HIER_EINVAL},
      {&HierTopo::B, INT_MAX, HIER_EUNSUPPORTED}, {&HierTopo::fa_max, -1, HIER_EINVAL},
      {&HierTopo::fl_max, INT_MAX, HIER_EUNSUPPORTED}, {&HierTopo::fg_max, -7, HIER_EINVAL},
  };
  HierMetaCounts cnt = {dev<int32_t>(21), dev<int32_t>(22), dev<int32_t>(23), dev<int32_t>(24),
                        dev<int32_t>(25)};
  for (const Bad& b : bad) {            // one bad field each: the call must stop at its check
    HierTopo x = good_topo();
    x.*(b.f) = b.v;
    EXPECT(hier_meta_count(&x, &cnt, nullptr), b.want);
  }
  HierTopo x = good_topo();
  x.labels = nullptr;                                              // labels mode, no labels
  EXPECT(hier_meta_build(&x, &out, nullptr), HIER_EINVAL);
  x = good_topo();
  x.use_membership = 1;                                            // membership arrays missing
  EXPECT(hier_meta_build(&x, &out, nullptr), HIER_EINVAL);
}

static HierFwdArgs good_fwd() {
  HierFwdArgs a;
  std::memset(&a, 0, sizeof(a));
  a.H = 24; a.D = 128; a.n_items = 0; a.scale = 0.088f; a.kv_rows = 37632;
  a.q = dev<uint16_t>(1); a.k = dev<uint16_t>(2); a.v = dev<uint16_t>(3); a.o = dev<uint16_t>(4);
  a.q_ss = a.k_ss = a.v_ss = a.o_ss = 3072;
  a.q_sh = a.k_sh = a.v_sh = a.o_sh = 128;
  a.tile_items = dev<int32_t>(5); a.tile_kv_idx = dev<int32_t>(6);
  a.tile_kv_mask = dev<uint32_t>(7); a.tile_blk_and = dev<uint32_t>(8);
  return a;
}

static void fwd_checks() {
  EXPECT(hier_attn_fwd(nullptr, nullptr), HIER_EINVAL);
  HierFwdArgs a = good_fwd();
  EXPECT(hier_attn_fwd(&a, nullptr), HIER_OK);                     // no items: nothing launched
  a = good_fwd(); a.D = 96;            EXPECT(hier_attn_fwd(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_fwd(); a.H = 0;             EXPECT(hier_attn_fwd(&a, nullptr), HIER_EINVAL);
  a = good_fwd(); a.n_items = -1;      EXPECT(hier_attn_fwd(&a, nullptr), HIER_EINVAL);
  a = good_fwd(); a.kv_rows = -3;      EXPECT(hier_attn_fwd(&a, nullptr), HIER_EINVAL);
  a = good_fwd(); a.v = nullptr;       EXPECT(hier_attn_fwd(&a, nullptr), HIER_EINVAL);
  a = good_fwd(); a.q = a.q + 1;       EXPECT(hier_attn_fwd(&a, nullptr), HIER_EINVAL);
  a = good_fwd(); a.k_ss = 3071;       EXPECT(hier_attn_fwd(&a, nullptr), HIER_EINVAL);
  a = good_fwd(); a.v_sh = -128;       EXPECT(hier_attn_fwd(&a, nullptr), HIER_EINVAL);
  a = good_fwd(); a.k_ss = 1ll << 40;  EXPECT(hier_attn_fwd(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_fwd(); a.k_ss = INT64_MAX - 7; EXPECT(hier_attn_fwd(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_fwd(); a.v_sh = INT64_MAX - 7; EXPECT(hier_attn_fwd(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_fwd(); a.kv_rows = INT_MAX; EXPECT(hier_attn_fwd(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_fwd(); a.n_items = INT_MAX; a.H = 1 << 20;
  EXPECT(hier_attn_fwd(&a, nullptr), HIER_EUNSUPPORTED);
}

static HierBwdArgs good_bwd() {
  HierBwdArgs a;
  std::memset(&a, 0, sizeof(a));
  a.H = 24; a.D = 128; a.scale = 0.088f; a.kv_rows = a.q_rows = 18816;
  a.q = dev<uint16_t>(1); a.k = dev<uint16_t>(2); a.v = dev<uint16_t>(3); a.o = dev<uint16_t>(4);
  a.dout = dev<uint16_t>(5); a.lse = dev<float>(6); a.delta = dev<float>(7);
  a.lse2 = dev<float>(8); a.dq = dev<uint16_t>(9); a.dk = dev<uint16_t>(10);
  a.dv = dev<uint16_t>(11);
  a.q_ss = a.k_ss = a.v_ss = a.o_ss = a.do_ss = a.dq_ss = a.dk_ss = a.dv_ss = 3072;
  a.q_sh = a.k_sh = a.v_sh = a.o_sh = a.do_sh = a.dq_sh = a.dk_sh = a.dv_sh = 128;
  a.lse_stride_h = 18816;
  a.tile_items = dev<int32_t>(12); a.tile_kv_idx = dev<int32_t>(13);
  a.tile_kv_mask = dev<uint32_t>(14); a.tile_blk_and = dev<uint32_t>(15);
  a.key_items = dev<int32_t>(16); a.key_q_idx = dev<int32_t>(17);
  a.key_q_mask = dev<uint32_t>(18); a.key_blk_and = dev<uint32_t>(19);
  return a;
}

static void bwd_checks() {
  EXPECT(hier_attn_bwd(nullptr, nullptr), HIER_EINVAL);
  HierBwdArgs a = good_bwd();
  EXPECT(hier_attn_bwd(&a, nullptr), HIER_OK);                     // no items: nothing launched
  a = good_bwd(); a.D = 32;            EXPECT(hier_attn_bwd(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_bwd(); a.n_key_items = -2;  EXPECT(hier_attn_bwd(&a, nullptr), HIER_EINVAL);
  a = good_bwd(); a.lse2 = nullptr;    EXPECT(hier_attn_bwd(&a, nullptr), HIER_EINVAL);
  a = good_bwd(); a.dk = a.dk + 3;     EXPECT(hier_attn_bwd(&a, nullptr), HIER_EINVAL);
  a = good_bwd(); a.do_sh = 12;        EXPECT(hier_attn_bwd(&a, nullptr), HIER_EINVAL);
  a = good_bwd(); a.q_ss = INT64_MAX - 7; EXPECT(hier_attn_bwd(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_bwd(); a.k_sh = INT64_MAX - 7; EXPECT(hier_attn_bwd(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_bwd(); a.n_ste_items = -1;  EXPECT(hier_attn_bwd(&a, nullptr), HIER_EINVAL);
  a = good_bwd(); a.n_ste_items = 4;   EXPECT(hier_attn_bwd(&a, nullptr), HIER_EINVAL);
  a = good_bwd(); a.n_ste_items = 4; a.ste_items = dev<int32_t>(20);
  a.ste_kv_idx = dev<int32_t>(21); a.ste_kv_mask = dev<uint32_t>(22);
  a.ste_kv_class = dev<int32_t>(23); a.ste_partial = dev<float>(24); a.ste_classes = 17;
  EXPECT(hier_attn_bwd(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_bwd(); a.tile_kv_class = dev<int32_t>(25);                // ste_partial missing
  EXPECT(hier_attn_bwd(&a, nullptr), HIER_EINVAL);
  a = good_bwd(); a.tile_kv_class = dev<int32_t>(25); a.n_ste_items = 1; a.ste_items = dev<int32_t>(20);
  a.ste_kv_idx = dev<int32_t>(21); a.ste_kv_mask = dev<uint32_t>(22);
  a.ste_kv_class = dev<int32_t>(23); a.ste_partial = dev<float>(24); a.ste_classes = 4;
  EXPECT(hier_attn_bwd(&a, nullptr), HIER_EINVAL);                   // both STE forms
  // the allocation-free entry point: its own workspace, its size limit
  a = good_bwd();
  EXPECT(hier_attn_bwd_noalloc(&a, nullptr), HIER_EINVAL);           // delta / lse2 given
  a.delta = nullptr; a.lse2 = nullptr; a.lse_stride_h = 1ll << 21;
  EXPECT(hier_attn_bwd_noalloc(&a, nullptr), HIER_EUNSUPPORTED);     // 2 x 24 x 2M floats
  a.lse_stride_h = INT64_MAX - 1;
  EXPECT(hier_attn_bwd_noalloc(&a, nullptr), HIER_EUNSUPPORTED);
  a.H = INT_MAX; a.lse_stride_h = INT64_MAX / 2;
  EXPECT(hier_attn_bwd_noalloc(&a, nullptr), HIER_EUNSUPPORTED);
  a.H = 0;
  EXPECT(hier_attn_bwd_noalloc(&a, nullptr), HIER_EINVAL);
}

static HierDeriveArgs good_derive() {
  HierDeriveArgs a;
  std::memset(&a, 0, sizeof(a));
  a.n_items = 189; a.n_groups = 49; a.rows = 18816; a.nq_max = 3; a.kv_len = 262144;
  a.P = 4; a.T = 21; a.L = 220; a.N = 2; a.KL = 5;
  a.items = dev<int32_t>(1); a.kv_idx = dev<int32_t>(2); a.kv_mask = dev<uint32_t>(3);
  a.ws = dev<void>(4); a.totals = dev<int64_t>(5);
  a.ws_bytes = hier_derive_workspace(&a);
  return a;
}

static void derive_checks() {
  if (hier_derive_workspace(nullptr) != -1) {
    std::printf("FAIL hier_derive_workspace(NULL) != -1\n");
    ++g_fail;
  }
  // workspace sizing over a grid of sizes: positive, monotone in each size
  const int items[] = {1, 7, 189, 378, 5000, 1 << 20};
  const int groups[] = {1, 3, 49, 98, 1000};
  const int rows[] = {1, 777, 18816, 37632, 92400, 1 << 24};
  const int frames[] = {1, 3, 6, 32};
  for (int ni : items)
    for (int ng : groups)
      for (int nr : rows)
        for (int nq : frames) {
          HierDeriveArgs a = good_derive();
          a.n_items = ni; a.n_groups = ng; a.rows = nr; a.nq_max = nq;
          const int64_t w = hier_derive_workspace(&a);
          a.rows = nr + 1;
          const int64_t w_more = hier_derive_workspace(&a);
          a.rows = nr; a.n_items = ni + 1;
          const int64_t w_items = hier_derive_workspace(&a);
          if (w <= 0 || w_more < w || w_items < w) {
            std::printf("FAIL workspace %d %d %d %d: %lld %lld %lld\n", ni, ng, nr, nq,
                        (long long)w, (long long)w_more, (long long)w_items);
            ++g_fail;
          }
        }
  HierDeriveArgs a = good_derive();
  a.n_groups = INT_MAX; a.nq_max = 32;                                // table too large
  (void)hier_derive_workspace(&a);
  EXPECT(hier_derive_count(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_derive(); a.n_items = INT_MAX; a.rows = INT_MAX;          // sizing stays in range
  (void)hier_derive_workspace(&a);
  EXPECT(hier_derive_count(nullptr, nullptr), HIER_EINVAL);
  a = good_derive(); a.n_groups = 0;   EXPECT(hier_derive_count(&a, nullptr), HIER_EINVAL);
  a = good_derive(); a.nq_max = 33;    EXPECT(hier_derive_count(&a, nullptr), HIER_EINVAL);
  a = good_derive(); a.kv_len = -1;    EXPECT(hier_derive_count(&a, nullptr), HIER_EINVAL);
  a = good_derive(); a.L = -220;       EXPECT(hier_derive_count(&a, nullptr), HIER_EINVAL);
  a = good_derive(); a.ws_bytes -= 1;  EXPECT(hier_derive_count(&a, nullptr), HIER_EINVAL);
  a = good_derive(); a.totals = nullptr; EXPECT(hier_derive_count(&a, nullptr), HIER_EINVAL);
  a = good_derive();                                                // pass 2 outputs missing
  EXPECT(hier_derive_build(&a, nullptr), HIER_EINVAL);
  a.key_items = dev<int32_t>(6); a.key_q_idx = dev<int32_t>(7);
  a.key_q_mask = dev<uint32_t>(8); a.key_blk_and = dev<uint32_t>(9);
  a.key_entries = 100;                                             // not a multiple of 64
  EXPECT(hier_derive_build(&a, nullptr), HIER_EINVAL);
  a.key_entries = 128; a.ste_entries = 64;                         // STE outputs missing
  EXPECT(hier_derive_build(&a, nullptr), HIER_EINVAL);
  a.ste_entries = -64;
  EXPECT(hier_derive_build(&a, nullptr), HIER_EINVAL);
  EXPECT(hier_derive_ste_classes(nullptr, nullptr, nullptr, nullptr), HIER_EINVAL);
  a = good_derive(); a.n_items = -1;
  EXPECT(hier_derive_ste_classes(&a, dev<int32_t>(10), dev<int32_t>(11), nullptr), HIER_EINVAL);
  a = good_derive(); a.items = nullptr;
  EXPECT(hier_derive_ste_classes(&a, dev<int32_t>(10), dev<int32_t>(11), nullptr), HIER_EINVAL);
}

static HierPrologueArgs good_prologue() {
  HierPrologueArgs a;
  std::memset(&a, 0, sizeof(a));
  a.S = 0; a.H = 24; a.D = 128; a.eps = 1e-6f;
  a.qx = dev<uint16_t>(1); a.kx = dev<uint16_t>(2); a.norm_q_w = dev<uint16_t>(3);
  a.norm_k_w = dev<uint16_t>(4); a.rope_cos = dev<float>(5); a.rope_sin = dev<float>(6);
  a.q_out = dev<uint16_t>(7); a.k_out = dev<uint16_t>(8);
  a.out_stride_s = 3072; a.out_stride_h = 128;
  return a;
}

static void prologue_checks() {
  EXPECT(hier_qkv_prologue(nullptr, nullptr), HIER_EINVAL);
  HierPrologueArgs a = good_prologue();
  EXPECT(hier_qkv_prologue(&a, nullptr), HIER_OK);                   // no tokens
  a = good_prologue(); a.D = 96;       EXPECT(hier_qkv_prologue(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_prologue(); a.S = -1;       EXPECT(hier_qkv_prologue(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_prologue(); a.H = INT_MAX;  EXPECT(hier_qkv_prologue(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_prologue(); a.kx = nullptr; EXPECT(hier_qkv_prologue(&a, nullptr), HIER_EINVAL);
  a = good_prologue(); a.out_stride_h = 129; EXPECT(hier_qkv_prologue(&a, nullptr), HIER_EINVAL);
  a = good_prologue(); a.cam = dev<uint16_t>(9); a.C = 11;
  EXPECT(hier_qkv_prologue(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_prologue(); a.S = INT_MAX;  EXPECT(hier_qkv_prologue(&a, nullptr), HIER_EUNSUPPORTED);
  a = good_prologue(); a.S = 1000; a.out_stride_s = INT64_MAX - 7;
  EXPECT(hier_qkv_prologue(&a, nullptr), HIER_EUNSUPPORTED);
}

static void page_and_frame_checks() {
  EXPECT(hier_kv_append(nullptr, nullptr), HIER_EINVAL);
  HierPageArgs p;
  std::memset(&p, 0, sizeof(p));
  p.H = 24; p.D = 128; p.n_rows = 1; p.pool_rows = 100;   // one row: checks run
  p.k_src = dev<uint16_t>(1); p.v_src = dev<uint16_t>(2); p.dst_rows = dev<int32_t>(3);
  p.k_pool = dev<uint16_t>(4); p.v_pool = dev<uint16_t>(5);
  p.k_src_ss = p.v_src_ss = p.pool_ss = 3072; p.k_src_sh = p.v_src_sh = p.pool_sh = 128;
  HierPageArgs b = p; b.D = 4;         EXPECT(hier_kv_append(&b, nullptr), HIER_EINVAL);
  b = p; b.n_rows = -1;                EXPECT(hier_kv_append(&b, nullptr), HIER_EINVAL);
  b = p; b.v_pool = nullptr;           EXPECT(hier_kv_append(&b, nullptr), HIER_EINVAL);
  b = p; b.k_src = b.k_src + 1;        EXPECT(hier_kv_append(&b, nullptr), HIER_EINVAL);
  b = p; b.pool_sh = 12;               EXPECT(hier_kv_append(&b, nullptr), HIER_EINVAL);
  b = p; b.H = INT_MAX;                EXPECT(hier_kv_append(&b, nullptr), HIER_EUNSUPPORTED);

  EXPECT(hier_frame_attn(nullptr, nullptr), HIER_EINVAL);
  HierFrameAttnArgs f;
  std::memset(&f, 0, sizeof(f));
  f.B = 1; f.Lq = 1; f.Lk = 1; f.H = 24; f.D = 128; f.n_block = 3; f.local_attn = 21;  // one query: checks run
  f.scale = 0.088f;
  f.q = dev<uint16_t>(1); f.k = dev<uint16_t>(2); f.v = dev<uint16_t>(3); f.o = dev<uint16_t>(4);
  f.q_frame = dev<int32_t>(5); f.k_frame = dev<int32_t>(6);
  HierFrameAttnArgs g = f; g.D = 80;   EXPECT(hier_frame_attn(&g, nullptr), HIER_EUNSUPPORTED);
  g = f; g.n_block = 0;                EXPECT(hier_frame_attn(&g, nullptr), HIER_EINVAL);
  g = f; g.Lq = -1;                    EXPECT(hier_frame_attn(&g, nullptr), HIER_EINVAL);
  g = f; g.q_frame = nullptr;          EXPECT(hier_frame_attn(&g, nullptr), HIER_EINVAL);
  g = f; g.o = g.o + 2;                EXPECT(hier_frame_attn(&g, nullptr), HIER_EINVAL);
  g = f; g.k_sh = 7;                   EXPECT(hier_frame_attn(&g, nullptr), HIER_EINVAL);
  g = f; g.H = 70000;                  EXPECT(hier_frame_attn(&g, nullptr), HIER_EUNSUPPORTED);
  g = f; g.B = INT_MAX; g.Lq = INT_MAX;
  EXPECT(hier_frame_attn(&g, nullptr), HIER_EUNSUPPORTED);
}

// The checks hand the library stand-in device addresses: they must never
// reach a GPU.
extern "C" int hipGetDeviceCount(int* count);

static void misc_checks() {
  EXPECT(hier_gated_residual(nullptr, nullptr), HIER_EINVAL);
  HierGateArgs ga;
  std::memset(&ga, 0, sizeof(ga));
  ga.rows = 1; ga.dim = 64; ga.rows_per_gate = 1;
  ga.x = dev<uint16_t>(1); ga.y = dev<uint16_t>(2); ga.gate = dev<uint16_t>(3); ga.out = dev<uint16_t>(4);
  ga.x_ss = ga.y_ss = ga.gate_ss = ga.out_ss = 64;
  HierGateArgs gb = ga; gb.dim = 12;      EXPECT(hier_gated_residual(&gb, nullptr), HIER_EINVAL);
  gb = ga; gb.rows_per_gate = 0;          EXPECT(hier_gated_residual(&gb, nullptr), HIER_EINVAL);
  gb = ga; gb.y_ss = 8;                   EXPECT(hier_gated_residual(&gb, nullptr), HIER_EINVAL);
  gb = ga; gb.gate = nullptr;             EXPECT(hier_gated_residual(&gb, nullptr), HIER_EINVAL);
  gb = ga; gb.out = gb.out + 1;           EXPECT(hier_gated_residual(&gb, nullptr), HIER_EINVAL);
  gb = ga; gb.rows = INT64_MAX / 2;       EXPECT(hier_gated_residual(&gb, nullptr), HIER_EUNSUPPORTED);
  gb = ga; gb.rows = 0;                   EXPECT(hier_gated_residual(&gb, nullptr), HIER_OK);

  EXPECT(hier_ste_reduce(nullptr, nullptr), HIER_EINVAL);
  HierSteReduceArgs sr;
  std::memset(&sr, 0, sizeof(sr));
  sr.H = 24; sr.P = 4; sr.T = 21; sr.L = 220; sr.N = 2; sr.KL = 5; sr.classes = 4;
  sr.partial = dev<float>(1); sr.out = dev<float>(2);
  sr.stride_h = (int64_t)(4 * 21 * 220 + 21 * 2 * 5) * 4;
  HierSteReduceArgs sb = sr; sb.classes = 3;   EXPECT(hier_ste_reduce(&sb, nullptr), HIER_EINVAL);
  sb = sr; sb.classes = 17;                    EXPECT(hier_ste_reduce(&sb, nullptr), HIER_EINVAL);
  sb = sr; sb.stride_h -= 1;                   EXPECT(hier_ste_reduce(&sb, nullptr), HIER_EINVAL);
  sb = sr; sb.T = INT_MAX;                     EXPECT(hier_ste_reduce(&sb, nullptr), HIER_EINVAL);
  sb = sr; sb.out = nullptr;                   EXPECT(hier_ste_reduce(&sb, nullptr), HIER_EINVAL);

  EXPECT(hier_membership_from_logits(nullptr, nullptr), HIER_EINVAL);
  HierMembershipArgs ma;
  std::memset(&ma, 0, sizeof(ma));
  ma.T = 21; ma.N = 2; ma.P = 4; ma.B = 7; ma.n = 3; ma.fl_max = 10;
  ma.logits = dev<float>(1); ma.la_frame = dev<int32_t>(2); ma.membership = dev<uint8_t>(3);
  ma.global_only = dev<uint8_t>(4); ma.q_active = dev<uint8_t>(5); ma.local_active = dev<uint8_t>(6);
  HierMembershipArgs mb = ma; mb.B = 6;        EXPECT(hier_membership_from_logits(&mb, nullptr), HIER_EINVAL);
  mb = ma; mb.P = INT_MAX;                     EXPECT(hier_membership_from_logits(&mb, nullptr), HIER_EINVAL);
  mb = ma; mb.la_frame = nullptr;              EXPECT(hier_membership_from_logits(&mb, nullptr), HIER_EINVAL);
  mb = ma; mb.T = INT_MAX; mb.B = INT_MAX; mb.n = 1;
  EXPECT(hier_membership_from_logits(&mb, nullptr), HIER_EINVAL);

  EXPECT(hier_merge_hub_lists(nullptr, nullptr), HIER_EINVAL);
  HierMergeArgs mg;
  std::memset(&mg, 0, sizeof(mg));
  mg.n_groups = 2; mg.n_src = 3; mg.rows = 1000; mg.rows_per_item = 128;
  mg.items = dev<int32_t>(1); mg.kv_idx = dev<int32_t>(2); mg.kv_mask = dev<uint32_t>(3);
  mg.blk_and = dev<uint32_t>(4); mg.acc = dev<uint32_t>(5); mg.src_item = dev<int32_t>(6);
  mg.src_group = dev<int32_t>(7); mg.src_shift = dev<int32_t>(8); mg.out_off = dev<int64_t>(9);
  mg.out_cap = dev<int32_t>(10); mg.group_desc = dev<int32_t>(11);
  mg.group_item_off = dev<int32_t>(12); mg.out_items = dev<int32_t>(13);
  HierMergeArgs mh = mg; mh.rows_per_item = 100;   EXPECT(hier_merge_hub_lists(&mh, nullptr), HIER_EINVAL);
  mh = mg; mh.rows = 0;                            EXPECT(hier_merge_hub_lists(&mh, nullptr), HIER_EINVAL);
  mh = mg; mh.n_groups = INT_MAX; mh.rows = INT_MAX;
  EXPECT(hier_merge_hub_lists(&mh, nullptr), HIER_EINVAL);
  mh = mg; mh.acc = nullptr;                       EXPECT(hier_merge_hub_lists(&mh, nullptr), HIER_EINVAL);
  mh = mg; mh.src_from = dev<int32_t>(14);         EXPECT(hier_merge_hub_lists(&mh, nullptr), HIER_EINVAL);
  mh = mg; mh.src_nbits = dev<int32_t>(15);        EXPECT(hier_merge_hub_lists(&mh, nullptr), HIER_EINVAL);
  mh = mg; mh.n_groups = 0;                        EXPECT(hier_merge_hub_lists(&mh, nullptr), HIER_OK);

  EXPECT(hier_trim_key_lists(nullptr, nullptr), HIER_EINVAL);
  HierTrimArgs tr;
  std::memset(&tr, 0, sizeof(tr));
  tr.n_items = 5; tr.items = dev<int32_t>(1); tr.kv_mask = dev<uint32_t>(2);
  tr.out_items = dev<int32_t>(3);
  HierTrimArgs ts = tr; ts.n_items = -1;            EXPECT(hier_trim_key_lists(&ts, nullptr), HIER_EINVAL);
  ts = tr; ts.kv_mask = nullptr;                   EXPECT(hier_trim_key_lists(&ts, nullptr), HIER_EINVAL);
  ts = tr; ts.out_items = nullptr;                 EXPECT(hier_trim_key_lists(&ts, nullptr), HIER_EINVAL);
  ts = tr; ts.n_items = 0; ts.items = nullptr;     EXPECT(hier_trim_key_lists(&ts, nullptr), HIER_OK);
}

int main() {
  int n_dev = 0;
  if (hipGetDeviceCount(&n_dev) == 0 && n_dev > 0) {
    std::printf("skipped: a GPU is visible\n");
    return 0;
  }
  if (std::strncmp(hier_version(), "hierattn", 8) != 0) {
    std::printf("FAIL hier_version: %s\n", hier_version());
    ++g_fail;
  }
  meta_checks();
  fwd_checks();
  bwd_checks();
  derive_checks();
  prologue_checks();
  page_and_frame_checks();
  misc_checks();
  std::printf("host checks done: %d failed\n", g_fail);
  return g_fail;
}
