/*
 * hierattn.h -- C ABI of the MI355X (gfx950) hierarchical group attention.
 *
 * Plain C: no HIP, torch or C++ types in any signature.  Every pointer named
 * "device" is a HIP device pointer owned by the caller; the library never
 * allocates or frees caller memory.  Every call is asynchronous on the given
 * stream (a hipStream_t passed as void*, NULL = the null stream) and returns
 * 0 on success or a negative HIER_E* code; hier_last_error() then returns a
 * thread-local message.
 *
 * Token orders used below (reference definitions):
 *   full sequence  [P*T*L agents p-major | T*N*KL locals time-major | T*KG global]
 *                  multics/models/hier_masks.py:549-571
 *   cached pool    [P*fa*L agents p-major | N*fl*KL locals g-major | fg*KG global]
 *                  multics/models/kernels/hier_segmented_attention.py:247-258
 *   cached queries [P*n*L agents | n*N*KL locals | n*KG global]
 *                  multics/models/attention.py:474-476
 */
#ifndef HIERATTN_H
#define HIERATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  HIER_OK = 0,
  HIER_EINVAL = -1,      /* invalid argument        -> ValueError          */
  HIER_EUNSUPPORTED = -2,/* unsupported shape/dtype -> NotImplementedError */
  HIER_ELAUNCH = -3,     /* HIP launch/runtime error -> RuntimeError       */
  HIER_EINTERNAL = -4    /* violated internal invariant -> AssertionError  */
};

/* ------------------------------------------------------------------------ */
/* Topology of B independent temporal blocks (one cached call is B = 1; a    */
/* full-sequence forward is B = T / n).  All arrays are DEVICE pointers.     */
/* ------------------------------------------------------------------------ */
typedef struct HierTopo {
  int32_t P, N, L, KL, KG;          /* players, group slots, tokens per frame  */
  int32_t n_frames, n_block;        /* query frames per block, causal block n  */
  int32_t local_attn;               /* sliding window W in frames, -1 = none   */
  int32_t direct;                   /* same-group, same-block player edges     */
  int32_t no_local;                 /* K_L = 0 topology (hier_no_local_hub)    */
  int32_t use_membership;           /* membership/global_only (else labels)    */
  int32_t B;                        /* number of blocks                        */
  int32_t fa_max, fl_max, fg_max;   /* row pitch of the per-block frame arrays */
  int32_t T_mem;                    /* rows of membership / global_only        */
  /* per block */
  const int32_t* fa;                /* [B] agent frames per player stream      */
  const int32_t* fl;                /* [B] frames per local stream             */
  const int32_t* fg;                /* [B] global frames                       */
  const int32_t* agent_frames;      /* [B][P][fa_max] absolute frame ids, ascending */
  const int32_t* local_frames;      /* [B][N][fl_max]                          */
  const int32_t* global_frames;     /* [B][fg_max]                             */
  const uint8_t* local_active;      /* [B][N][fl_max] local slot active per cached frame */
  const int32_t* q_frames;          /* [B][n_frames] absolute query frames     */
  const int32_t* labels;            /* [B][n_frames][P] (labels mode)          */
  const uint8_t* q_active;          /* [B][n_frames][N]                        */
  const uint8_t* membership;        /* [T_mem][N][P] (membership mode)         */
  const uint8_t* global_only;       /* [T_mem][P]                              */
  /* addressing: token offset of frame fi of each stream, for the reference  */
  /* arrays (ref_*) and for the attention kernel's K/V pool (tile_*)         */
  const int32_t* ref_agent_base;    /* [B][P][fa_max]                          */
  const int32_t* ref_local_base;    /* [B][N][fl_max]                          */
  const int32_t* ref_global_base;   /* [B][fg_max]                             */
  const int32_t* tile_agent_base;   /* [B][P][fa_max]                          */
  const int32_t* tile_local_base;   /* [B][N][fl_max]                          */
  const int32_t* tile_global_base;  /* [B][fg_max]                             */
  /* query rows: first row and frame pitch of every stream (P + N + 1 per    */
  /* block; local entries unused when no_local)                              */
  const int32_t* ref_qbase;         /* [B][P+N+1]                              */
  const int32_t* tile_qbase;        /* [B][P+N+1]                              */
  int32_t ref_qstride[3];           /* frame pitch of agent / local / global rows */
  int32_t tile_qstride[3];
} HierTopo;

/* Per-segment counts written by hier_meta_count (DEVICE arrays).           */
/* Segment order inside a block follows _build_metadata:                    */
/* players (p, qrel), locals (qrel, g), global (qrel).                       */
typedef struct HierMetaCounts {
  int32_t* seg_count;      /* [B][n_seg] compact key count per segment        */
  int32_t* tiled_count;    /* [B][n_seg] kept Tiled128 slots (multiple of 128)*/
  int32_t* dense_count;    /* [B][n_seg] dense slots                          */
  int32_t* logical_count;  /* [B][n_seg] valid dense slots                    */
  int32_t* tile_count;     /* [B][P+N+1] union keys per stream, padded to 64  */
} HierMetaCounts;

/* Output arrays written by hier_meta_build.  Any group may be NULL to skip. */
typedef struct HierMetaOut {
  /* _build_metadata format (bit-exact), block b at offsets *_off[b]         */
  int32_t block_m;
  const int64_t* seg_prog_off;    /* [B] program offset of block b            */
  const int64_t* seg_kv_off;      /* [B] element offset of block b's matrix   */
  const int32_t* seg_max_k;       /* [B] MAX_K of block b                      */
  int32_t* seg_prog_qbase;        /* [sum programs]                            */
  int32_t* seg_prog_nq;
  int32_t* seg_prog_seg;
  int32_t* seg_kv_index;          /* [sum n_seg*MAX_K]                         */
  int32_t* seg_kv_count;          /* [B*n_seg]                                 */
  /* Tiled128 format (labels only, bit-exact)                                */
  const int64_t* tiled_prog_off;
  const int64_t* tiled_kv_off;
  const int32_t* tiled_max_k;
  int32_t* tiled_prog_qbase;
  int32_t* tiled_prog_nq;
  int32_t* tiled_prog_seg;
  int32_t* tiled_kv_index;
  uint8_t* tiled_kv_valid;
  int32_t* tiled_kv_count;
  /* attention-kernel tile list: per (block, stream) the ordered union of its */
  /* query frames' key lists with a per-key bitmask over query frames         */
  const int64_t* tile_kv_off;     /* [B][P+N+1] key offset of each stream     */
  const int32_t* tile_item_off;   /* [B][P+N+1] first work item of each stream */
  int32_t rows_per_item;          /* query rows per work item (multiple of 32) */
  int32_t* tile_kv_idx;           /* [sum tile_count] K/V pool token index     */
  uint32_t* tile_kv_mask;         /* [sum tile_count] visible-to-query-frame bits */
  uint32_t* tile_blk_and;         /* [sum tile_count / 64] AND of masks per 64 keys */
  int32_t* tile_items;            /* [n_items][8] work item descriptors        */
} HierMetaOut;

/* Pass 1: evaluate the hierarchical edge rule for every (segment, cached   */
/* frame run) and count.  Replaces the count half of _build_metadata         */
/* (multics/models/kernels/hier_segmented_attention.py:156-395), _pack_layout */
/* (hier_tiled_attention.py:182-241) and the cached/full-sequence Tiled128   */
/* builders (hier_tiled_attention.py:244-429, 474-655).                      */
int hier_meta_count(const HierTopo* topo, const HierMetaCounts* counts, void* stream);

/* Pass 2: fill the arrays sized from pass 1's counts (same references).     */
int hier_meta_build(const HierTopo* topo, const HierMetaOut* out, void* stream);

/* ------------------------------------------------------------------------ */
/* Backward lists derived on the device from a full-sequence tile list:     */
/* the key-major list of the dK / dV pass and the membership-STE list, bit  */
/* for bit the host builders transpose_tiles_host / ste_tiles_host of       */
/* multics_amd/metadata.py.  No reference counterpart: the reference's      */
/* backward is FlexAttention's autograd over its BlockMask                  */
/* (multics/models/attention.py:322-353, 367-434).                          */
/* ------------------------------------------------------------------------ */
typedef struct HierDeriveArgs {
  /* forward tile list (DEVICE) */
  int32_t n_items;          /* work items                                       */
  int32_t n_groups;         /* (block, stream) groups = items with row_start 0   */
  int32_t rows;             /* 1 + largest row / key index (queries = keys)      */
  int32_t nq_max;           /* largest frame count of a group (<= 32)            */
  int32_t kv_len;           /* entries of kv_idx / kv_mask                       */
  int32_t P, T, L, N, KL;   /* STE geometry (token order of the full sequence)   */
  const int32_t* items;     /* [n_items][8]                                      */
  const int32_t* kv_idx;
  const uint32_t* kv_mask;
  /* workspace (DEVICE, hier_derive_workspace bytes) and pass-1 results       */
  void* ws;
  int64_t ws_bytes;
  int64_t* totals;          /* DEVICE [8]: key-major entries, pairs, STE entries, */
                            /* STE items, error bits (1 token in two groups,      */
                            /* 2 key outside every group, 4 not whole key frames, */
                            /* 8 malformed items, 16 offset overflow)             */
  /* pass 2: sizes read back from totals, output arrays (DEVICE)              */
  int64_t key_entries, ste_entries;
  int32_t* key_items;       /* [n_items][8]                                      */
  int32_t* key_q_idx;       /* [key_entries]                                     */
  uint32_t* key_q_mask;
  uint32_t* key_blk_and;    /* [key_entries / 64]                                */
  int32_t* ste_items;       /* [totals[3]][8]                                    */
  int32_t* ste_kv_idx;      /* [ste_entries]                                     */
  uint32_t* ste_kv_mask;
  uint32_t* ste_blk_and;    /* [ste_entries / 64]                                */
  int32_t* ste_kv_class;    /* [ste_entries]                                     */
} HierDeriveArgs;

/* Workspace bytes for the sizes in args (ws may be NULL); -1 on NULL args.  */
int64_t hier_derive_workspace(const HierDeriveArgs* args);
/* Pass 1: groups, token map, run table, list sizes and offsets -> totals.   */
int hier_derive_count(const HierDeriveArgs* args, void* stream);
/* Pass 2: the two lists, their per-64 mask ANDs and their items.            */
int hier_derive_build(const HierDeriveArgs* args, void* stream);
/* Membership-STE class of every entry of the forward list (n_items, kv_len, */
/* P..KL, items, kv_idx, kv_mask of args; no workspace, no pass 1): g for a */
/* local-hub key of group g in a player group's list, p for a key of player */
/* p in a local-hub group's list, -1 for every other entry and for masks of */
/* 0 -- the selection of the STE list, kept in forward-list order; each    */
/* item writes the entries of its own range -- and item_first[i] = the      */
/* first 64-entry tile of item i's range holding a class (its tile count if */
/* none).  Inputs tile_kv_class / tile_ste_first of hier_attn_bwd.          */
int hier_derive_ste_classes(const HierDeriveArgs* args, int32_t* kv_class, int32_t* item_first,
                            void* stream);

/* Hub streams of a full-sequence tile list merged across temporal blocks:  */
/* the rows of G consecutive blocks of one local-hub slot (or of the global */
/* hub) become one group whose key list is the union of the G source lists, */
/* a key's mask bits of block b0 + j shifted by n * j.  Sources are given by */
/* one of their items (its list offset and padded size are read on the      */
/* device); each merged list goes, in key-row order, into its slot          */
/* [out_off, out_off + out_cap) of the same kv arrays, padded to 64 with    */
/* mask 0, with its per-64 mask ANDs; the group's items (rows split into    */
/* rows_per_item pieces) go to out_items at group_item_off.  acc is a       */
/* [n_groups][rows] uint32 workspace.  No reference counterpart (the        */
/* reference runs one program per segment: hier_tiled_attention.py:52-146). */
typedef struct HierMergeArgs {
  int32_t n_groups, n_src;
  int32_t rows;                    /* key rows (1 + largest key index)         */
  int32_t rows_per_item;
  const int32_t* items;            /* the built list's items                   */
  int32_t* kv_idx;                 /* the built list's arrays (sources read,   */
  uint32_t* kv_mask;               /* merged slots written)                    */
  uint32_t* blk_and;
  uint32_t* acc;                   /* [n_groups][rows] workspace               */
  const int32_t* src_item;         /* [n_src] an item of each source list      */
  const int32_t* src_group;        /* [n_src] merged group of each source      */
  const int32_t* src_shift;        /* [n_src] bit shift of its masks           */
  const int64_t* out_off;          /* [n_groups] slot offsets (multiples of 64) */
  const int32_t* out_cap;          /* [n_groups] slot capacities (multiples of 64) */
  const int32_t* group_desc;       /* [n_groups][4] qbase, qstride, qlen, frames */
  const int32_t* group_item_off;   /* [n_groups] first output item             */
  int32_t* out_items;              /* [sum items][8]                           */
  /* Optional per-source bit selection (both NULL: every source's whole     */
  /* mask): source i contributes bits [src_from[i], src_from[i] +           */
  /* src_nbits[i]) of its masks, moved down to bit 0 before the shift, so a  */
  /* player's last query frames can join a hub group under bits of their    */
  /* own (its group's items then take their rows from a row table: qstride  */
  /* -1 in group_desc).                                                     */
  const int32_t* src_from;         /* [n_src] first mask bit taken             */
  const int32_t* src_nbits;        /* [n_src] number of bits taken (1..32)     */
} HierMergeArgs;

int hier_merge_hub_lists(const HierMergeArgs* args, void* stream);

/* Work items with each key list cut to the 64-entry tiles that some row of */
/* the item can see: the new range runs from the first to the last such    */
/* tile (kv_off advances by whole tiles, kv_cnt is capped at the old end);  */
/* an item whose rows see no entry keeps its range.  A row's mask bit is    */
/* its frame (row_start + r) / qlen, or the row table's bit for items with  */
/* qstride -1 (row_table [rows][2] (token, bit), NULL if no item needs it). */
/* The entries dropped are masked for every row of the item, so every pass  */
/* over the cut list (forward, dQ, dK / dV) gives the same results while    */
/* copying and multiplying fewer tiles.  items and out_items may be the     */
/* same array.  No reference counterpart (the reference's kernels walk      */
/* each segment's whole padded list: hier_tiled_attention.py:52-146,        */
/* hier_segmented_attention.py:27-114).                                     */
typedef struct HierTrimArgs {
  int32_t n_items;
  int32_t reserved;
  const int32_t* items;            /* [n_items][8]                             */
  const uint32_t* kv_mask;         /* the list's masks                         */
  const int32_t* row_table;        /* [rows][2] or NULL                        */
  int32_t* out_items;              /* [n_items][8]                             */
} HierTrimArgs;

int hier_trim_key_lists(const HierTrimArgs* args, void* stream);

/* Membership-dependent topology arrays of a full-sequence membership        */
/* topology from soft membership logits, in one launch: membership =        */
/* logits > 0, global_only = in no group, and the query-frame / local-slot   */
/* activity (a group is active where it has a member), as                   */
/* _prepare_hier_membership_tensors derives them (multics/models/            */
/* hier_masks.py:127-193); written into the arrays a HierTopo points at, so */
/* the lists of new logits are rebuilt with no host round trip.            */
typedef struct HierMembershipArgs {
  int32_t T, N, P;                 /* frames, group slots, players             */
  int32_t B, n;                    /* temporal blocks, frames per block (B*n = T) */
  int32_t fl_max;                  /* local-slot columns per block             */
  const float* logits;             /* [T][N][P] fp32 (DEVICE)                  */
  const int32_t* la_frame;         /* [B][fl_max] frame of each column, < 0 = padding */
  uint8_t* membership;             /* [T][N][P]                                */
  uint8_t* global_only;            /* [T][P]                                   */
  uint8_t* q_active;               /* [B][n][N]                                */
  uint8_t* local_active;           /* [B][N][fl_max]                           */
} HierMembershipArgs;

int hier_membership_from_logits(const HierMembershipArgs* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Q/K/V layout prologue: camera-pose Q/K adapter, RMSNorm over all heads,  */
/* gain and RoPE fused into one pass that writes the attention layout.       */
/* Replaces SelfAttention._project_self_attn_qkv after the three GEMMs      */
/* (multics/models/attention.py:355-365, 307-320, 231-242) and rope_apply    */
/* (multics/models/rope.py:248-254).                                         */
/* ------------------------------------------------------------------------ */
typedef struct HierPrologueArgs {
  int32_t S, H, D;                 /* tokens, heads, head dim (64 or 128)     */
  float eps;                       /* RMSNorm epsilon                          */
  const uint16_t* qx;              /* [S][H*D] bf16 q(x) (with bias)           */
  const uint16_t* kx;              /* [S][H*D] bf16 k(x)                       */
  const uint16_t* vx;              /* [S][H*D] bf16 v(x), copied to the layout */
  const uint16_t* cam;             /* [S][C] bf16 camera tokens or NULL        */
  const uint16_t* w_cam_q;         /* [H*D][C] bf16 cam_q.weight or NULL       */
  const uint16_t* w_cam_k;         /* [H*D][C] bf16                            */
  int32_t C;                       /* camera feature width (12)                */
  const uint16_t* norm_q_w;        /* [H*D] bf16 RMSNorm gains                 */
  const uint16_t* norm_k_w;
  const float* rope_cos;           /* [S][D/2] fp32 (from the complex freqs)   */
  const float* rope_sin;           /* [S][D/2]                                 */
  uint16_t* q_out;                 /* bf16 outputs at [s*stride_s + h*stride_h + d] */
  uint16_t* k_out;
  uint16_t* v_out;
  int64_t out_stride_s, out_stride_h;
} HierPrologueArgs;

int hier_qkv_prologue(const HierPrologueArgs* args, void* stream);

/* Backward of hier_qkv_prologue's q and k outputs: the autograd of the     */
/* camera add, RMSNorm, gain and RoPE (attention.py:355-365, 307-320,        */
/* 231-242; rope.py:248-254), recomputed in fp32 from the forward's inputs: */
/*   dz = rotate(d_out, -theta), dy = dz * w, dw += dz * bf16(a * r),        */
/*   d_proj = r * dy - r^3 * a * sum(dy * a) / dim,                         */
/* a = the projection plus the bf16 camera product, r = its inverse RMS.    */
/* Writes d_proj (bf16 [S][H*D], the gradient of q(x) / k(x) and of the     */
/* camera adapter's output) and per wave one fp32 row of gain-gradient      */
/* partials ([hier_qk_prologue_bwd_waves][H*D], to be summed by the caller; */
/* the camera-weight gradient is d_proj^T . cam, a plain GEMM).  Model dims */
/* that are multiples of 512 up to 4096, head dim 64 or 128.                */
typedef struct HierPrologueBwdArgs {
  int32_t S, H, D;
  float eps;
  int32_t C;                       /* camera feature width (12) if cam          */
  int32_t tokens_per_wave;         /* consecutive tokens per wave (>= 1)        */
  const uint16_t* qx;              /* [S][H*D] bf16 forward inputs              */
  const uint16_t* kx;
  const uint16_t* cam;             /* [S][C] bf16 camera tokens or NULL         */
  const uint16_t* w_cam_q;         /* [H*D][C] bf16                             */
  const uint16_t* w_cam_k;
  const uint16_t* norm_q_w;        /* [H*D] bf16 RMSNorm gains                  */
  const uint16_t* norm_k_w;
  const float* rope_cos;           /* [S][D/2] fp32                             */
  const float* rope_sin;
  const uint16_t* dq;              /* bf16 gradient of q, (s,h,d) at s*dq_ss + h*dq_sh + d */
  const uint16_t* dk;
  int64_t dq_ss, dq_sh, dk_ss, dk_sh;
  uint16_t* dqx;                   /* [S][H*D] bf16 gradient of q(x)            */
  uint16_t* dkx;
  float* dw_q_partial;             /* [waves][H*D] fp32                         */
  float* dw_k_partial;
} HierPrologueBwdArgs;

/* Rows of each dw_*_partial buffer for args (S, tokens_per_wave); -1 if invalid. */
int hier_qk_prologue_bwd_waves(const HierPrologueBwdArgs* args);
int hier_qk_prologue_bwd(const HierPrologueBwdArgs* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Block-sparse frame-causal flash attention forward over the tile list.    */
/* Replaces _segmented_attn_fwd / _tiled128_fwd launches                     */
/* (hier_segmented_attention.py:27-114, 474-500; hier_tiled_attention.py:52-146, */
/* 766-795) and the FlashInfer / varlen calls (hier_paged_attention.py:238-267, */
/* hier_packed_attention.py:230-242).  Rows with no visible key are 0.       */
/* ------------------------------------------------------------------------ */
typedef struct HierFwdArgs {
  int32_t H, D;                    /* heads, head dim (64 or 128)              */
  int32_t n_items;                 /* work items (tile_items rows)             */
  float scale;                     /* softmax scale (1/sqrt(D))                */
  int32_t kv_rows;                 /* rows addressable in k / v (> every key index) */
  int32_t reserved;                /* must be 0                                */
  const uint16_t* q;               /* bf16, element (s,h,d) at s*q_ss + h*q_sh + d */
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;                     /* bf16 output, rows not covered are untouched */
  float* lse;                      /* [H][S_q] log-sum-exp (natural log) or NULL */
  int64_t q_ss, q_sh, k_ss, k_sh, v_ss, v_sh, o_ss, o_sh;
  int64_t lse_stride_h;            /* elements between heads of lse            */
  const int32_t* tile_items;       /* from hier_meta_build                      */
  const int32_t* tile_kv_idx;
  const uint32_t* tile_kv_mask;
  const uint32_t* tile_blk_and;
  /* Items whose qstride is -1 take their rows from this table instead:     */
  /* row r of such an item is the pair (token, mask bit) at                 */
  /* row_table[2 * (qbase + r)] (r = row_start ..), so one item can hold rows */
  /* of several streams against one key list.  NULL if no item does.        */
  const int32_t* row_table;
} HierFwdArgs;

int hier_attn_fwd(const HierFwdArgs* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Backward of hier_attn_fwd: dQ, dK, dV.  Replaces the autograd backward of */
/* the Flex path the training forward differentiates through               */
/* (attention.py:322-353, 367-434; hier_masks.py:690-719).                  */
/* Two launches on `stream`: a query-major pass over the forward tile list   */
/* (dQ; also writes -delta = -rowsum(dO * O) and lse2 = lse * log2(e) into  */
/* the caller's workspace) and a key-major pass over the transposed list     */
/* (dK, dV), so every gradient row is written by exactly one workgroup: no   */
/* atomics, deterministic.  Gradient rows that no item covers are untouched; */
/* key rows of a key item that no query sees are written as 0.             */
/* ------------------------------------------------------------------------ */
typedef struct HierBwdArgs {
  int32_t H, D;                    /* heads, head dim (64 or 128)              */
  int32_t n_items;                 /* query-major items (forward tile list)    */
  int32_t n_key_items;             /* key-major items (transposed tile list)   */
  float scale;                     /* softmax scale of the forward             */
  int32_t kv_rows;                 /* rows addressable in k / v                */
  int32_t q_rows;                  /* rows addressable in q / dout             */
  int32_t reserved;                /* must be 0                                */
  const uint16_t* q;               /* bf16 inputs of the forward               */
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;               /* bf16 forward output                      */
  const uint16_t* dout;            /* bf16 gradient of the output              */
  const float* lse;                /* [H][.] natural-log LSE from the forward  */
  float* delta;                    /* [H][.] workspace, written                */
  float* lse2;                     /* [H][.] workspace, written                */
  uint16_t* dq;                    /* bf16 gradients                           */
  uint16_t* dk;
  uint16_t* dv;
  int64_t q_ss, q_sh, k_ss, k_sh, v_ss, v_sh, o_ss, o_sh, do_ss, do_sh;
  int64_t dq_ss, dq_sh, dk_ss, dk_sh, dv_ss, dv_sh;
  int64_t lse_stride_h;            /* elements between heads of lse / delta / lse2 */
  const int32_t* tile_items;       /* forward (query-major) tile list          */
  const int32_t* tile_kv_idx;
  const uint32_t* tile_kv_mask;
  const uint32_t* tile_blk_and;
  const int32_t* key_items;        /* transposed (key-major) tile list: items  */
  const int32_t* key_q_idx;        /* describe key rows, lists hold query rows */
  const uint32_t* key_q_mask;      /* bit f: the query sees key frame f        */
  const uint32_t* key_blk_and;
  /* Optional membership STE (n_ste_items > 0): a query-major list holding   */
  /* only the keys whose edge to the query row is gated by one membership    */
  /* bit -- local-hub keys of group g for player-p rows, player-p keys for   */
  /* local-hub rows of group g, both at the query frame -- with per key the  */
  /* class c (g for player rows, p for local-hub rows).  The pass adds      */
  /* dS = P (dP - delta) over each row's keys of class c into                */
  /* ste_partial[h][row][c] (fp32, row stride ste_classes <= 16: classes    */
  /* >= ste_classes are dropped; zero-initialised by the caller); rows of    */
  /* other items are untouched.                                              */
  int32_t n_ste_items;
  int32_t ste_classes;
  const int32_t* ste_items;
  const int32_t* ste_kv_idx;
  const uint32_t* ste_kv_mask;
  const int32_t* ste_kv_class;
  float* ste_partial;              /* [H][ste_rows][ste_classes]               */
  int64_t ste_stride_h;            /* elements between heads of ste_partial    */
  /* Optional membership STE inside the dQ pass (instead of an STE list,    */
  /* n_ste_items must then be 0): the class of every entry of the forward    */
  /* list (-1 or >= 16 = no gating bit) and per item the first 64-entry tile */
  /* of its list with a class (both from hier_derive_ste_classes).  The dQ   */
  /* pass adds dS over each row's entries of class c into                    */
  /* ste_partial[h][row][c] and writes it for every row of every item.       */
  const int32_t* tile_kv_class;
  const int32_t* tile_ste_first;   /* [n_items]                                */
  /* Key-major items whose kstride (item[1]) is -1 take their key rows from  */
  /* this table: row r is the pair (token, key-frame bit) at                 */
  /* key_row_table[2 * (kbase + r)], so one item can hold the keys of        */
  /* several streams against one query list (hier_merge_hub_lists run on the */
  /* key-major list).  NULL if no key item does.                            */
  const int32_t* key_row_table;
} HierBwdArgs;

int hier_attn_bwd(const HierBwdArgs* args, void* stream);

/* hier_attn_bwd without a caller workspace: no counterpart in the reference.  */
/* For callers that cannot allocate device memory (code under HIP graph      */
/* capture, tight training loops, harnesses that forbid hipMalloc).  Same    */
/* arguments, kernels and results as hier_attn_bwd, except that delta and    */
/* lse2 must be NULL: they live in a 16 MiB device array of the library      */
/* (2 x H x lse_stride_h <= 4M floats, else HIER_EUNSUPPORTED), one copy per */
/* GPU, held until the process ends and cleared by each call.  The call      */
/* allocates nothing; calls that overlap on one GPU race on that array.      */
int hier_attn_bwd_noalloc(const HierBwdArgs* args, void* stream);

/* Membership-STE sums of hier_attn_bwd's ste_partial reduced over heads and */
/* rows into the gradient layout of the membership logits [T][N][P]:        */
/*   out[t][g][p] = sum_h sum_{l<L} partial[h][(p*T + t)*L + l][g]           */
/*                + sum_h sum_{k<KL} partial[h][P*T*L + (t*N + g)*KL + k][p] */
/* (full-sequence token order).  Deterministic (fixed summation order); no   */
/* counterpart in the reference, whose membership has no gradient.  Every    */
/* player and local-hub row of partial must be written (the dQ pass writes  */
/* every row of every item).                                                */
typedef struct HierSteReduceArgs {
  int32_t H, P, T, L, N, KL;
  int32_t classes;                 /* row stride of partial (>= P and N, <= 16) */
  const float* partial;            /* [H][rows][classes]                       */
  int64_t stride_h;                /* elements between heads of partial        */
  float* out;                      /* [T][N][P] fp32                           */
} HierSteReduceArgs;

int hier_ste_reduce(const HierSteReduceArgs* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Paged KV cache append: copy the new K/V rows of a cached block into their */
/* pool rows.  Replaces the per-stream rolling-cache writes and the per-call */
/* pool concatenation of the cached path (attention.py:90-228, 605-666;     */
/* hier_segmented_attention.py:458-469): every stream-frame owns a fixed    */
/* page of pool rows, a re-run block overwrites its pages (refresh in place) */
/* and a frame older than the window is overwritten by the newest one (the  */
/* eviction), so no row ever moves.  Rows whose destination is outside      */
/* [0, pool_rows) are skipped.                                              */
/* ------------------------------------------------------------------------ */
typedef struct HierPageArgs {
  int32_t H, D;                    /* heads, head dim (multiple of 8)          */
  int32_t n_rows;                  /* source rows                              */
  int32_t pool_rows;               /* rows of each pool                        */
  const uint16_t* k_src;           /* bf16 rows of the block                   */
  const uint16_t* v_src;
  int64_t k_src_ss, k_src_sh, v_src_ss, v_src_sh;
  const int32_t* dst_rows;         /* [n_rows] DEVICE: pool row of each source row */
  uint16_t* k_pool;                /* bf16 [pool_rows] rows                    */
  uint16_t* v_pool;
  int64_t pool_ss, pool_sh;        /* strides of both pools                    */
} HierPageArgs;

int hier_kv_append(const HierPageArgs* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Frame-window attention of the action branches' cached attention: the     */
/* F.scaled_dot_product_attention(attn_mask=...) calls of                   */
/* blocks.py:307 (mouse temporal self-attention, one token per frame) and   */
/* blocks.py:374 (keyboard cross-attention), whose boolean mask is          */
/*   visible(i, j) = k_frame[j] / n_block <= q_frame[i] / n_block           */
/*                   and (local_attn == -1 or q_frame[i] - k_frame[j] < local_attn) */
/* (blocks.py:303-306, 366-372).  Rows that see no key are written as 0.    */
/* Element (b, s, h, d) of q / k / v / o is at b*_sb + s*_ss + h*_sh + d.   */
/* ------------------------------------------------------------------------ */
typedef struct HierFrameAttnArgs {
  int32_t B, Lq, Lk, H, D;         /* batch, queries, keys, heads, head dim (64 or 128) */
  int32_t n_block;                 /* frames per block (>= 1)                  */
  int32_t local_attn;              /* window in frames, -1 = unbounded         */
  float scale;                     /* softmax scale (1/sqrt(D))                */
  const uint16_t* q;               /* bf16                                     */
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t q_sb, q_ss, q_sh, k_sb, k_ss, k_sh, v_sb, v_ss, v_sh, o_sb, o_ss, o_sh;
  const int32_t* q_frame;          /* [Lq] DEVICE: frame of each query         */
  const int32_t* k_frame;          /* [Lk] DEVICE: frame of each key           */
} HierFrameAttnArgs;

int hier_frame_attn(const HierFrameAttnArgs* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Gated residual of the DiT block after self-attention,                    */
/*   out = x + gate * y,                                                    */
/* replacing GateModule.forward(x, gate_msa, self_attn_out)                 */
/* (multics/models/blocks.py:31-35, applied at blocks.py:661, 668).  One     */
/* gate row serves rows_per_gate consecutive rows (a frame's tokens share   */
/* their player-frame's gate_msa, blocks.py:604-616).  bf16 throughout,     */
/* bit-identical to torch's bf16 expression (product rounded to bf16, then  */
/* the sum); out may equal x.  Row strides in elements.                     */
/* ------------------------------------------------------------------------ */
typedef struct HierGateArgs {
  int64_t rows;                    /* rows of x / y / out                      */
  int32_t dim;                     /* channels per row (multiple of 8)         */
  int32_t rows_per_gate;           /* rows sharing one gate row (>= 1)         */
  const uint16_t* x;               /* bf16 [rows][x_ss]                        */
  const uint16_t* y;               /* bf16 [rows][y_ss]                        */
  const uint16_t* gate;            /* bf16 [rows / rows_per_gate][gate_ss]     */
  uint16_t* out;                   /* bf16 [rows][out_ss]                      */
  int64_t x_ss, y_ss, gate_ss, out_ss;
} HierGateArgs;

int hier_gated_residual(const HierGateArgs* args, void* stream);

/* Last error message of the calling thread ("" if none).                    */
const char* hier_last_error(void);

/* Library version string and the offload target it was built for.         */
const char* hier_version(void);

#ifdef __cplusplus
}
#endif

#endif /* HIERATTN_H */
