/*
 * aoship_internal.h — launch parameter blocks shared between the C ABI (host) and the kernels.
 *
 * Device data layouts:
 *
 *   int4 base matrix W[out][in] ("q4 tiles"), out % 32 == 0, in % 64 == 0, G = in / 64,
 *   RB = out / 32 row blocks:
 *     qt[((rb * G + g) * 64 + l) * 4 + j], l in 0..63, j in 0..3
 *        = shuffle(Wp[rb*32 + l%32][g*8 + 4*(l/32) + j])
 *     where Wp is the MLX word (8 nibbles, low nibble first) and shuffle reorders the nibbles
 *     to (n0, n2, n4, n6, n1, n3, n5, n7) so that masking with 0x000F000F after a shift of
 *     4p yields the natural pair (n[2p], n[2p+1]). One row block and group is one contiguous
 *     1 KiB chunk: a wave reads it with one 16-byte load per lane.
 *     sb[(rb * G + g) * 32 + n] = f16 scale | f16 bias << 16 for row rb*32+n, group g.
 *
 *   LoRA module: A[rpad][in] and B[out][rpad] bfloat16 row-major, rank zero-padded to rpad, a
 *   multiple of 16. The prefill GEMMs read a second copy of B in fragment order,
 *   Bf[out / 32][rpad / 8][32][8]: element (o, j) at ((o / 32) * (rpad / 8) + j / 8) * 256 +
 *   (o % 32) * 8 + j % 8, so that the 8 columns j0 .. j0 + 7 of 32 consecutive rows are one
 *   contiguous 512-byte run (one MFMA operand load of 32 lanes) instead of 32 rows' slices.
 *
 *   Activations: bfloat16 [T][features] row-major.
 */
#ifndef AOSHIP_INTERNAL_H
#define AOSHIP_INTERNAL_H

#include <stdint.h>

#include "../../include/aoship.h"

#define AOS_MAX_MODULES 7
enum { MOD_Q = 0, MOD_K, MOD_V, MOD_O, MOD_GATE, MOD_UP, MOD_DOWN };

#define AOS_MAX_ADAPTERS 4096
#define AOS_DECODE_MAX_T 32
#ifndef AOS_GEMV_LDS_MAX
#define AOS_GEMV_LDS_MAX (32 * 1024) /* dynamic LDS budget of one GEMV workgroup (measured) */
#endif
#define AOS_SHRINK_GROUPS_PER_WAVE 2

/* Arrival counting over n workgroups in two levels: groups of AOS_ARRIVE_GROUP arrivals count
 * into a counter of their own, and the last of each group into the top counter (same-address
 * device-scope atomics are performed one after another). Counter words for n arrivals: the top
 * line and one line per group, 32 words (128 bytes) a line. */
#define AOS_ARRIVE_GROUP 32u
#ifndef AOS_ARRIVE_STRIDE
#define AOS_ARRIVE_STRIDE 32u /* words between counters */
#endif
#define AOS_ARRIVE_WORDS(n)                                                                             \
  (AOS_ARRIVE_STRIDE *                                                                                    \
   ((uint32_t)(n) <= AOS_ARRIVE_GROUP ? 1u : 1u + ((uint32_t)(n) + AOS_ARRIVE_GROUP - 1u) / AOS_ARRIVE_GROUP))

typedef struct {
  int out, in, G, RB;
  const uint32_t *qt;
  const uint32_t *sb;
} aos_q4_dev;

/* Per-module view of the bound adapter table. */
typedef struct {
  int n;        /* table length */
  int rpad;     /* padded rank (multiple of 16), 0 if no adapter has this module */
  const uint16_t *const *A; /* device array [n] of device pointers (NULL = absent) */
  const uint16_t *const *B;
  const uint16_t *const *Bf; /* B in fragment order (the prefill GEMMs' copy) */
  const float *scale;       /* device [n] alpha / rank */
} aos_lora_tab;

/* Adapter plan of one layer call (T <= 32 tokens), built once from the rings:
 * the union of adapters used by the tokens (ascending index), each token's coefficient
 * scale * q / 32767 for each adapter of the union (0 when the token does not use it), and, for
 * up to AOS_PLAN_NPTR pointer tables named at the build, the union's row pointers in each
 * (ptr[k][u] = table_k[list[u]], so that a reader needs one load rather than two dependent ones).
 * Entries at u >= U are stale. */
#define AOS_PLAN_MAXU 256
#define AOS_PLAN_NPTR 4
typedef struct {
  int U;
  int pad[3];
  uint16_t list[AOS_PLAN_MAXU];
  float coef[AOS_DECODE_MAX_T][AOS_PLAN_MAXU];
  uint64_t ptr[AOS_PLAN_NPTR][AOS_PLAN_MAXU];
} aos_plan;

typedef struct {
  const aoship_ring_t *rings;
  int T;
  int n;                 /* bound table length */
  const uint8_t *bound;  /* [n] 1 = adapter bound for this layer */
  const float *scale;    /* [n] */
  aos_plan *plan;
  const uint16_t *const *ptab[AOS_PLAN_NPTR]; /* device pointer tables [n] listed per union slot
                                                 into plan->ptr (NULL: not listed) */
} aos_plan_params;

/* ---- router ---- */
typedef struct {
  int n, d, T, k;
  float tau, eps, bias;
  const float *features;
  const float *router_w;
  const float *priors_in;
  float *priors_out;
  const uint64_t *stable_id;
  const uint8_t *allowed;
  aoship_ring_t *rings;
  int32_t *status;
  /* router extras, each NULL when off */
  const uint8_t *scope;        /* [n] 0 = prior replaced by -1e9 (scope hint) */
  const uint64_t *tie_key;     /* [n] adaptive mode: rank of (breaker, stable_id, index) */
  const uint8_t *post_allowed; /* [n] decision policy: 1 = the adapter passes the policy sets */
  int post_max;                /* decision policy: max adapters per token, -1 = no cap */
  const uint16_t *active_ids;  /* [n] ring index for a decision index */
  const float *strengths;      /* [n] gate scaling by decision index */
  uint8_t *hashes;             /* [T][96] decision hashes (input, output, combined) */
  const uint32_t *hash_extra;  /* [16] reasoning hash words 0-7, backend identity hash words 8-15 */
  int hash_reasoning, hash_backend;
  aoship_decision_t *decisions; /* [T] entropy and candidates */
} aos_route_params;

/* ---- LoRA shrink for T <= 32 tokens: S[t][col] = sum_i A_row(col)[i] x[t][i], float32 ----
 * Row col = (adapter slot u, rank row j) with u = col / rpad. In "all" mode slot u is adapter u
 * of the table (no rings needed); otherwise slot u is plan->list[u] (the call's union). Up to 3
 * modules sharing x in one launch. The grid is (row blocks of 32 summed over the modules, ks);
 * one extra workgroup (blockIdx.x == n_rb_total) builds the plan when plan_build is set. */
typedef struct {
  const uint16_t *x; /* [T][in] bf16 */
  int T, in;
  int nmod;
  aos_lora_tab tab[3];
  float *S[3];       /* [T][s_stride] float32 per module */
  int s_stride[3];
  int n_rb[3];       /* row blocks per module */
  int all_mode;      /* 1: rows over every table slot; 0: over plan->list */
  const aos_plan *plan;
  int ks;            /* K splits across workgroups */
  int lds_bytes;
  float *part;       /* [rb_total][ks][16 * 64] */
  uint32_t *counters;/* [rb_total] zero between launches */
  aos_plan_params plan_build; /* used when plan_build.plan != NULL */
  const uint16_t *zero_row;   /* device zeros, read by lanes without an adapter row */
  /* fused launch, per-producer lines: once row block r's S is stored, its finishing workgroup
   * raises lines[32 r] to gen; the plan workgroup raises lines[32 rb_total] once the plan is
   * stored (NULL: no lines) */
  uint32_t *lines;
  uint32_t gen;
} aos_shrink_params;

/* ---- decode GEMV ---- */
typedef struct {
  aos_q4_dev w0, w1;  /* w1 used in SwiGLU mode (up), w0 = gate or the single matrix */
  const uint16_t *x;  /* [T][in] bf16 */
  int T;
  int ks;             /* workgroups per row block (split K) */
  int waves;          /* waves per workgroup: 4 or 8 */
  int wr;             /* row blocks per workgroup (divides waves): wave w takes row block
                         wr * rbg + w % wr of the workgroup's row-block group rbg and K piece
                         w / wr of the workgroup's K split; all of them share the staged x */
  int nrbg;           /* row-block groups: ceil(RB / wr); workgroup (rbg, ksi) of the grid */
  int lds_bytes;      /* dynamic LDS: x staging + group sums, or the wave reduction */
  int has_expand;     /* 1: the K-split workgroups of each row block add the LoRA expand */
  /* LoRA expand: coef(t, u) * S[t][col(u) + j] . B_list[u][row][j] over the plan's union */
  aos_lora_tab tab0, tab1;
  const float *S0, *S1;   /* [T][s_stride] float32 */
  int s_stride0, s_stride1;
  int s_all;              /* 1: S columns indexed by adapter, 0: by union slot */
  const aos_plan *plan;
  int pk0, pk1, pkh;      /* 1 + the plan's pointer table listing tab0.B, tab1.B, htab.A rows
                           * (0: looked up through plan->list and the table) */
  const uint16_t *zero_row;
  /* outputs */
  uint16_t *y;        /* [T][out] bf16 (plain) or h (SwiGLU) */
  float *yf;          /* plain mode: [T][out] float32 instead of y when not NULL */
  float *part;        /* [RB][ks][NA * NV * 64] */
  uint32_t *counters; /* [RB] zero between launches */
  /* fused launch (aos_launch_gemv_fused): the shrink that produces S0 / S1 (and the plan) runs
   * in the first workgroups of the same grid. Either every producer raises a line of its own
   * (pre_lines: n_pre_lines lines; the plan's is line plan_line, -1 when the plan comes from an
   * earlier launch) and each GEMV workgroup waits for the plan's line before loading its expand's
   * B rows and for every line before loading S; or (sync) the last of the sync_target producers
   * to finish raises one ready flag per GEMV workgroup, which waits for its own flag before its
   * expand. NULL sync and pre_lines: S and the plan come from earlier launches. */
  const uint32_t *pre_lines;
  int n_pre_lines;
  int plan_line;
  uint32_t *sync;     /* producer arrivals, AOS_ARRIVE_WORDS(sync_target) words; zero between launches */
  uint32_t *flags;    /* this matrix's ready flags [nrbg * ks * 32], one per workgroup and 128-byte line */
  uint32_t sync_target;
  uint32_t gen;       /* this launch's generation: a ready flag equal to it is raised */
  uint32_t *timeout;  /* set to 1 if a wait gave up (the launch still ends) */
  /* SwiGLU mode, fused launch (wr == 1): the down projection's LoRA shrink over this row block's
   * 32 rows of h, hpart[rb][t][col] = sum_r h[t][32 rb + r] A_down(col)[32 rb + r] for the plan's union
   * columns col < U * htab.rpad (NULL: not formed) */
  aos_lora_tab htab;
  float *hpart;
  int hstride;
  /* one-launch decode, gate/up (wr == 1): h and its shrink partials go out device-coherent, and each row
   * block's finisher counts itself into hdone (AOS_ARRIVE_WORDS(RB) words); the last of the RB
   * raises n_hflags flag lines
   * (hflags, one per later workgroup that reads h) to gen */
  uint32_t *hdone;
  uint32_t *hflags;
  uint32_t n_hflags;
} aos_gemv_params;

/* The sum of those partials over the row blocks, in row-block order: S[t][col] for col <
 * U * rpad, values_per_wg (= AOS_HSUM_V) consecutive (t, col) values per workgroup. */
#define AOS_HSUM_V 4
typedef struct {
  const float *hpart; /* [RB][T][stride] */
  int RB, T, stride, rpad;
  const aos_plan *plan;
  float *S;           /* [T][stride] */
  int values_per_wg;
  int coherent;       /* 1: hpart was written by this launch (device-scope loads) */
  uint32_t *lines;    /* fused launch, per-producer lines: workgroup b raises lines[32 b] to gen once
                         its sums are stored (NULL: no lines) */
  uint32_t gen;
} aos_hsum_params;

/* A shrink and the GEMVs that consume its S in one launch: workgroups [0, n_pre) run the shrink
 * (row block b % pre_rows, K split b / pre_rows; pre_rows counts the plan workgroup), workgroup
 * n_pre + r the GEMV of matrix i for r in [wg_end[i - 1], wg_end[i]) (n = 1 in SwiGLU mode).
 * gp[i].sync = sync, gp[i].flags = flags + 32 * wg_end[i - 1], gp[i].sync_target = n_pre. */
typedef struct {
  aos_shrink_params sp;
  aos_gemv_params gp[3];
  int wg_end[3];
  int n;
  int n_pre, pre_rows;
  int hsum;           /* 1: the first workgroups run hs (pre_rows = n_pre) instead of the shrink sp */
  aos_hsum_params hs;
  uint32_t *sync;     /* producer arrivals, AOS_ARRIVE_WORDS(n_pre) words (counted hand-off) */
  uint32_t *flags;    /* [n_cons * 32] (counted hand-off) */
  uint32_t n_cons;    /* wg_end[n - 1] */
  uint32_t gen;       /* generation the producers raise their lines / the flags to (nonzero) */
  uint32_t *lines;    /* per-producer hand-off: n_lines lines (pre_rows for a shrink, n_pre for the
                         sums), the same as sp.lines / hs.lines and every gp[i].pre_lines; NULL:
                         counted hand-off through sync and flags */
  int n_lines;
} aos_gemv_fused_params;

/* The decode MLP (1-2 tokens) in one launch: workgroups [0, gu.n_pre) run the x shrink and the
 * plan, the next gu.n_cons the gate/up GEMV (h and the h shrink's partials, device-coherent), the
 * next dn.n_pre sum those partials once every row block of h is done (their line of hflags), and
 * the last dn.n_cons run the down GEMV, which stream their weights first and stage h once it is
 * complete (their line of hflags), then wait for the h shrink's S as any fused consumer does.
 * gu.gen == dn.gen: the launch's generation. */
typedef struct {
  aos_gemv_fused_params gu, dn;
  uint32_t *hflags; /* [dn.n_pre + dn.n_cons] lines of 32 words */
} aos_decode_mlp_params;

/* Routing from features and the fused gate/up launch in one grid: workgroups [0, rp.T) route
 * one token each (the plain router), then fp's producers (the x shrink; its plan workgroup waits
 * for route_flag to equal fp.gen before reading the rings) and fp.gp[0]'s gate/up GEMV
 * workgroups. */
#define AOS_ROUTE_PARTS_MAXN 64 /* adapters up to which a token's priors are split over workgroups */
typedef struct {
  aos_route_params rp;
  aos_gemv_fused_params fp;
  uint32_t *route_done; /* router arrivals, zero between launches (the last router resets it) */
  uint32_t *route_flag; /* raised to fp.gen by the last router, on a line of its own */
  /* rparts > 1 (rp.n <= AOS_ROUTE_PARTS_MAXN): each token's priors are computed by rparts
   * workgroups, one wave per adapter (workgroup r: adapters 4 r .. 4 r + 3), stored to rpri[t][a]
   * device-coherently and counted on the token's line of rpart_ctr; the last of them routes the
   * token. rparts == 1: one workgroup per token computes every prior and routes. */
  int rparts;
  uint32_t *rpart_ctr;  /* [T] lines of 32 words, zero between launches */
  float *rpri;          /* [T][AOS_ROUTE_PARTS_MAXN] */
} aos_route_gu_params;

/* The decode MLP of one token, with its routing when rp is set, in one launch (aoship_mlp1.hip).
 * nwg = two workgroups per CU, all resident at once (LDS holds at most two), 8 waves each.
 * Waves 0-3 stream an even share of the gate/up units (row block rb, group g; unit rb * G + g, in
 * order) over all 4 nwg of them; waves 4-7 load their workgroup's share of the down matrix's
 * units into LDS at the start and multiply it with h once h is complete. The first of waves 4-7
 * also route the token (one wave per adapter's prior, the last of them routes) and form the x
 * shrink S for every adapter (a wave per 32-column tile and K piece). Every value one wave hands
 * to another is a 64-bit word (payload | gen << 32) stored device-coherently: the reader loads
 * it until the stamp equals this launch's generation, so no producer waits for its stores. A row
 * block's partial sums (gate/up or down) are summed by the wave holding its last unit (its
 * owner), over the waves before it in order; the owner adds the LoRA expand (for gate/up formed
 * ahead by otherwise idle waves, ex), and a gate/up owner forms h and its rows' part of the down
 * shrink (hpart). The down shrink S_h is summed over the
 * gate/up row blocks by one wave per column. The tagged buffers sit in the layer's flag memory
 * (zero at rest, cleared when a given-up wait is reset). */
#define AOS_MLP1_MAXN 64 /* adapters in the layer's table */
#define AOS_MLP1_MAXR 64 /* padded rank of each module */
#define AOS_MLP1_MAX_DU 20 /* down units per wave */
#define AOS_MLP1_LDS_MAX (80 * 1024) /* two workgroups per CU */
typedef struct {
  aos_q4_dev wg, wu, wd;     /* gate, up, down */
  const uint16_t *x;         /* [H] bf16 */
  uint16_t *y;               /* [H] bf16 */
  const aoship_ring_t *ring_in; /* the token's ring, when it is not routed in this launch */
  int route;                 /* 1: routed in this launch by rp (the plain router, one token) */
  aos_route_params rp;
  int n;                     /* adapter table length */
  const uint8_t *bound;      /* [n] */
  const float *scale;        /* [n] */
  aos_lora_tab tg, tu, td;   /* LoRA tables of gate, up, down */
  const uint16_t *zero_row;  /* >= 256 zero bytes */
  int nwg;
  int d_units_max;           /* most down units one workgroup holds */
  int doff;                  /* LDS offset of the down units */
  int lds_bytes;
  int x_tiles_g, x_tiles_u, x_ks; /* x shrink: 32-column tiles of gate and of up, K pieces */
  int hc;                    /* h-shrink columns per gate/up row block in hpart (8 * td.rpad) */
  /* tagged exchange words */
  uint64_t *gpart;           /* [4 nwg][64] gate (lanes 0-31) / up (32-63) partials handed on */
  uint64_t *dpart;           /* [4 nwg][32] down partials handed on */
  uint64_t *htag;            /* [I] h (bf16 in the payload) */
  uint64_t *hpart;           /* [RB_gate][hc] */
  uint64_t *ex;              /* [RB_gate][64] LoRA expand of gate (words 0-31) and up (32-63) */
  uint64_t *sh;              /* [hc] S_h */
  uint64_t *spart;           /* [(x_tiles_g + x_tiles_u) x_ks][32] */
  uint64_t *sx;              /* [n tg.rpad + n tu.rpad] S of every adapter: gate's, then up's */
  uint64_t *pri;             /* [n] priors */
  uint64_t *ringt;           /* [10] the ring's words */
  uint32_t gen;
  uint32_t *timeout;         /* set to 1 if a wait gave up (the launch still ends) */
} aos_mlp1_params;

/* q, k and v (or any n <= 3 matrices with the same x, T and waves) in one launch: matrix i owns
 * workgroups [wg_end[i - 1], wg_end[i]) of a 1-D grid, wg_end[i] - wg_end[i - 1] = RB_i * ks_i;
 * entries past n repeat wg_end[n - 1]. */
typedef struct {
  aos_gemv_params p[3];
  int wg_end[3];
  int n;
} aos_gemv3_params;

/* ---- prefill path (T > 32 tokens) ----
 * Tokens are grouped by adapter set before the GEMMs: a stable sort by a hash of each token's
 * active adapter set (ties by token index) gives perm[p] = the token at sorted position p. The
 * GEMMs run over 128-token tiles of the sorted order; each tile's LoRA work covers only the
 * adapters its own tokens use (the tile union, ascending adapter index). */
#define AOS_PREFILL_MAX_T 4096
#define AOS_GEMM_BM 128 /* tokens per tile */
#define AOS_TILE_U_MAX 1024 /* a tile's union: at most 128 tokens x 8 ring slots */
#define AOS_XE_COLS 512     /* union columns from which a tile's gate/up expand runs in the expand launch */

/* Group plan: the sort, then for each tile mt its union tu[mt] <= tu_cap, list[mt][u], the
 * coefficients coef[p][u] = sum over sorted token p's active ring slots naming list[mt][u] of
 * scale * q / 32767 (ring order), and per module the union's A and B pointers (NULL for an adapter
 * without the module). */
typedef struct {
  const aoship_ring_t *rings;
  int T, n;
  const uint8_t *bound;    /* [n] */
  const float *scale;      /* [n] */
  int tu_cap;              /* slots tabulated per tile (>= min(n, AOS_TILE_U_MAX)) */
  uint16_t *perm;          /* [T] */
  int *tu;                 /* [mtiles] */
  uint16_t *list;          /* [mtiles][tu_cap] */
  float *coef;             /* [T][tu_cap], rows in sorted order */
  int nmod;
  aos_lora_tab tab[3];
  const uint16_t **ap, **bp; /* [nmod][mtiles][tu_cap] */
} aos_gplan_params;

/* Tile shrink: for module i of a tile, S[p][c] = sum_k x[perm[p]][k] A_{list[u]}[j][k] over the
 * tile's union columns c = u * rpad_i + j, K split into ks slices; once every slice of a (tile,
 * column set) has stored its partial sums, each slice sums its share of the rows over the slices
 * in order and stores SA[p][off_i(mt) + c] = bf16(coef[p][u] * S) with off_i(mt) = sum over
 * modules i' < i of tu[mt] * rpad_i'. One workgroup per (K slice, set of four 32-column blocks,
 * tile), the K slice fastest: the slices that meet are consecutive workgroups. */
typedef struct {
  const uint16_t *x;       /* [T][in] activations in token order, or sorted order when !perm */
  const uint16_t *perm;    /* [T] or NULL (rows already in sorted order) */
  int T, in;
  int nmod;
  int rpad[3];
  const int *tu;
  const float *coef;
  int tu_cap;
  const uint16_t *const *ap; /* [nmod][mtiles][tu_cap] */
  int mtiles, csets, ks;   /* grid: mtiles x csets x ks */
  float *part;             /* [mtiles][ks][128][s_stride] float32 */
  uint32_t *counters;      /* [mtiles * csets], zero at rest */
  uint32_t *flags;         /* [mtiles * csets] lines of 32 words: the slices' meeting point */
  uint32_t gen;            /* raised to by the last slice of a (tile, column set) */
  uint32_t *timeout;       /* set when a wait gave up */
  uint16_t *SA;            /* [T][s_stride] bf16, sorted rows */
  int s_stride;            /* >= sum over modules of tu_cap * rpad_i, multiple of 64 */
  const uint16_t *zero_row;
  int am_tu;               /* > 0: tiles with tu >= am_tu are the adapter-major shrink's */
} aos_tshrink_params;

/* Adapter-major LoRA shrink: the alternative to the tile shrink when tile unions are much wider
 * than the adapters a token routes to (tokens that do not cluster). Users of adapter a: the
 * sorted positions p with a nonzero coefficient for a (union slot u of p's tile), in chunks of 128.
 * aos_amplan (one launch after the group plan) lists them: users[a * T + k] = (p << 16) | u for
 * k < count[a]; chunk c of the launch, ctab[c] = (a << 16) | (j << 8) | nu, is the j-th chunk of
 * adapter a, users[a * T + 128 j + r] for r < nu, adapters in index order; ctab[c] = 0 for the
 * unused tail up to cb (users of one adapter in no particular order: each user's sums depend on its own row
 * only); its other workgroups zero, in each SA buffer zb[], the entries of the tile's union columns
 * that no user covers (coefficient 0). Only tiles with tu >= am_tu take part (the tile shrink,
 * given the same am_tu, skips them). The last plan workgroup to finish builds ctab from the counts
 * and resets count[] and done[0] (both zero at rest). aos_amshrink, per chunk c, column set cs of the adapter's
 * columns (modules in order, rpad_i each) and K slice kz:
 * S[r][col] = sum_k x[row(p)][k] A_i,a[j][k] (row(p) = perm[p], or p without a permutation),
 * SA[p][off_i(tile(p)) + u * rpad_i + j] = bf16(coef[p][u] * S), off_i as in the tile shrink;
 * with ks > 1 slices each slice stores float32 partials and the reduce launch (reduce = 1, grid
 * cb x csets) sums them in slice order. */
#define AOS_AM_MAX_N 1024 /* adapters the adapter-major shrink takes */
#define AOS_AM_TU 8       /* union size (adapters) from which a prefill tile's shrinks run adapter-major */
typedef struct {
  uint16_t *SA;
  int s_stride, nmod;
  int rpad[3];
} aos_am_zero;

typedef struct {
  int T, n, tu_cap, cb, am_tu;
  const int *tu;
  const uint16_t *list;    /* [mtiles][tu_cap] */
  const float *coef;       /* [T][tu_cap] */
  uint32_t *count;         /* [n], zero at rest */
  uint32_t *done;          /* [1], zero at rest */
  uint32_t *ctab;          /* [cb] */
  uint32_t *users;         /* [n][T] */
  int nz;
  aos_am_zero zb[2];
  /* for the adapter-major expand (NULL / 0: none): per tile the users' range of each union slot
   * in users[a] ((base << 8) | count, tiles of the lists), the slot of each adapter (0xffff: none;
   * tiles with tu >= xam_tu, n <= AOS_XAM_MAX_N), and the tiles with tu >= xam_tu in order, their
   * count in xl[mtiles] */
  uint32_t *tinfo;         /* [mtiles][tu_cap] */
  uint16_t *inv;           /* [mtiles][n] */
  uint32_t *xl;            /* [mtiles + 1] */
  int xam_tu;
} aos_amplan_params;

/* Adapter-major gate/up expand of the tiles with tu >= xam_tu (in the order of xl, in ranges of
 * AOS_XAM_RT tiles; the expand launch skips them): for each range, module m and 32-row block r0,
 * d[p][o] = sum over the adapters a of p in index order of sum_j SA[p][off_m + u_a rpad_m + j]
 * B_m,a[o][j], accumulated in LDS and stored into xd in the expand launch's accumulator order.
 * The list launch (list = 1, grid = ranges) gathers each range's users in adapter order and cuts
 * them into chunks of at most 128 of one adapter (ct[c] = (first entry << 15) | (a << 8) | users,
 * nch[r] chunks, ct[nch] = 0), each chunk's local rows in rlp; it records each user's entry
 * cidx[a][k] = r * AOS_XAM_RT * 1024 + entry, where the x shrink writes the user's SA row (gate
 * then up columns) into SAc, the rows the expand reads. */
#define AOS_XAM_MAX_N 128
#define AOS_XAM_RT 4
#define AOS_XAM_TU 32 /* union size (adapters) from which a tile's gate/up expand runs adapter-major */
#define AOS_XAM_CT (AOS_XAM_RT * 8 + AOS_XAM_MAX_N + 4) /* chunks of a range at most, and the spare one */
typedef struct {
  int T, n, tu_cap, mtiles, RB;
  const int *tu;
  const uint32_t *tinfo;
  const uint16_t *inv;
  const uint32_t *xl;
  const uint32_t *users;   /* [n][T] */
  uint16_t *rlp;           /* [ranges][AOS_XAM_CT][128]: each chunk's users' local rows, the spare row
                              (AOS_XAM_RT * 128) past them and in the chunk after the last */
  uint32_t *ct;            /* [ranges][AOS_XAM_CT] */
  uint32_t *nch;           /* [ranges] */
  uint32_t *cidx;          /* [n][T] */
  const uint16_t *SAc;     /* [ranges][AOS_XAM_RT * 1024][rpad[0] + rpad[1]] */
  int rpad[2];             /* gate and up, equal: a multiple of 16 up to 64 */
  const uint16_t *const *Bf[2];
  const uint16_t *zero;    /* >= 64 zero elements */
  float *xd;
  int list;
} aos_amx_params;

typedef struct {
  const uint16_t *x;       /* [T][in] */
  const uint16_t *perm;    /* [T] or NULL */
  int T, in, nmod, tu_cap, ks, cb, csets; /* grid: ks x cb x csets (reduce: cb x csets) */
  int setw;                /* columns of a set: 64 (2-wave workgroups) or 128; csets = ceil(sum of
                              rpad_i / setw) */
  int rpad[3];
  const uint16_t *const *A[3]; /* per module: [n] device A pointers (NULL: adapter without it) */
  const int *tu;
  const float *coef;
  const uint32_t *ctab, *users; /* ctab[c] = (a << 16) | (j << 8) | users in the chunk (0: unused) */
  uint16_t *SA;
  int s_stride;
  float *part;             /* [ks][cb][csets][128][128] float32 when ks > 1 */
  const uint16_t *zero_row;
  int reduce;
  /* users of tiles with tu >= xam_tu (the adapter-major expand's) also go to the compact copy:
   * SAc[cidx[a][k]][col], col over the adapter's columns (NULL: none) */
  const uint32_t *cidx;    /* [n][T], parallel to users */
  uint16_t *SAc;
  int xam_tu;
} aos_amshrink_params;

/* int4 GEMM with the LoRA expand over the tile union: y[p][o] = sum_k x[p][k] w[o][k] +
 * sum_c SA[p][off + c] B_{list[u]}[o][c - u * rpad] (the expand as extra K steps of 64 union
 * columns), for the sorted rows p of each tile; SwiGLU mode computes gate (w0) and up (w1) and
 * writes (g * sigmoid(g)) * u. x rows are read through in_perm (NULL: sorted order) and y rows
 * written through out_perm (NULL: sorted order). */
typedef struct {
  aos_q4_dev w0, w1;
  const uint16_t *x;  /* [T][in] */
  const uint16_t *in_perm, *out_perm;
  int T;
  int mb, nb;         /* token tiles, weight blocks (set by the launcher for its kernel shape) */
  int rpad0, rpad1;   /* modules of w0 / w1 (0: no adapter has it) */
  int mod0;           /* module index of w0 in the plan's tables (w1: mod0 + 1) */
  const int *tu;
  const uint16_t *const *bp; /* [nmod][mtiles][tu_cap] */
  int tu_cap, mtiles;
  const uint16_t *SA; /* [T][sa_stride] bf16 */
  int sa_stride;
  int sa_mod_before;  /* modules of the shrink before mod0 (their columns come first) */
  int rpad_before[2]; /* their padded ranks */
  const uint16_t *zero; /* 16 zero bytes */
  uint16_t *y;        /* [T][out] */
  /* The LoRA shrink in the same launch (s_cols > 0): the launch's first mb * nbs workgroups
   * compute SA = bf16(coef * x . A^T) over each tile's union columns of module mod0 (and mod0 + 1
   * in SwiGLU mode) from the same token tiles, store it device-coherently and raise the tile's
   * line; the tile's GEMM workgroups wait for that line before their expand. s_cols is the larger
   * module's column count at the widest union (tu_cap * rpad); nbs is set by the launcher. */
  int s_cols, nbs;
  const uint16_t *const *ap; /* [nmod][mtiles][tu_cap] A pointers of the plan */
  const float *coef;         /* [T][tu_cap], sorted rows */
  uint16_t *sa_out;          /* == SA */
  uint32_t *sa_ctr;          /* [mtiles] arrival counters, zero at rest */
  uint32_t *sa_lines;        /* [mtiles] lines of 32 words, raised to gen */
  uint32_t gen;
  uint32_t *timeout;         /* set when a wait gave up */
  /* Stream-K (sk_nwg > 0): sk_nwg workgroups, the device's resident capacity for the kernel shape,
   * share the tasks' K groups evenly (aos_gemm_sk_slots); sk_part holds one slot of partial sums
   * per workgroup (aos_gemm_sk_slot_floats floats), sk_lines one line of 32 words per workgroup. */
  int sk_nwg;
  float *sk_part;
  uint32_t *sk_lines;
  /* SwiGLU mode: the LoRA expand of each tile whose union spans xe_cols or more columns of its
   * wider module (tu * max(rpad0, rpad1)) ran in an expand launch of its own (aos_xexp_params),
   * whose gate and up sums this launch adds before the activation instead of expanding itself.
   * xd: [2][mtiles][RB][4 sub-tiles][4][64 lanes][4] float32 (module, tile, 32-row block, the
   * accumulator's registers 4 q .. 4 q + 3 of each lane); NULL: every tile expands here. */
  const float *xd;
  int xe_cols;
} aos_gemm_params;

/* The expand launch of a SwiGLU prefill GEMM: for each tile with tu * rmax >= xe_cols and each
 * module m (0 gate, 1 up), xd[m] = SA . B^T over the tile's union columns of that module (g[m]
 * describes module m as the only module of a single-matrix expand), in the layout the GEMM reads. */
typedef struct {
  aos_gemm_params g[2];
  float *xd;
  int xe_cols, rmax;
  int xam_tu;              /* > 0: tiles with tu >= xam_tu are the adapter-major expand's */
} aos_xexp_params;

/* Where a launch goes: its stream and, when profiling, the HIP events the dispatch itself
 * records at kernel start and end (hipExtLaunchKernelGGL). */
typedef struct {
  void *stream;
  void *ev_start;
  void *ev_stop;
} aos_launch_ctx;

/* ---- full decoder step (embedding, norms, RoPE + KV cache, attention) ---- */
#define AOS_ATTN_MAX_HD 256
typedef struct {
  const int32_t *ids; /* [T] */
  int T, H, vocab;
  const uint32_t *q4;     /* [vocab][H / 8] MLX 4-bit rows, or NULL */
  const uint16_t *s16;    /* [vocab][H / 64] float16 scales */
  const uint16_t *b16;    /* [vocab][H / 64] float16 biases (NULL = 0) */
  const uint16_t *bf16;   /* [vocab][H] bfloat16 rows when q4 is NULL */
  float *hidden;          /* [T][H] float32 */
  int32_t *status;        /* set to 1 when an id is out of range (that row is zero) */
} aos_embed_params;

typedef struct {
  float *hidden;          /* [T][H] float32 residual stream */
  const uint16_t *add;    /* [T][H] bf16 added to hidden first, or NULL */
  const float *w;         /* [H] norm weight */
  float eps;
  int T, H;
  uint16_t *out;          /* [T][H] bf16 normalised */
} aos_norm_params;

typedef struct {
  const uint16_t *q, *k, *v; /* [T][nh*hd], [T][nkv*hd], [T][nkv*hd] bf16 projections */
  const float *bq, *bk, *bv; /* biases or NULL */
  const float *inv_freq;     /* [hd / 2] */
  int T, nh, nkv, hd, offset, max_seq;
  float *qr;                 /* [T][nh][hd] float32, rotated */
  uint16_t *kc, *vc;         /* [nkv][max_seq][hd] bf16 caches of this layer */
} aos_rope_params;

typedef struct {
  const float *q;            /* [T][nh][hd] rotated */
  uint16_t *kc, *vc;         /* [nkv][max_seq][hd] (written only with rope_fused) */
  int T, nh, nkv, hd, offset, max_seq;
  int splits, chunk;         /* key positions per split (multiple of 64) */
  float scale;
  float *part;               /* [T][nh][splits][hd + 2]: acc, running max, sum */
  uint16_t *out;             /* [T][nh * hd] bf16 */
  /* splits > 1: the last wave of (token, head) to finish merges the splits; counters [T][nh]
   * are zero between launches (that wave resets its own) */
  uint32_t *counters;
  /* rope_fused (T == 1): q, k and v come as the bf16 projections below; the attention applies
   * the biases and RoPE itself, uses the current token's key and value from LDS and appends them
   * to the cache (kv heads once each); q above is unused */
  int rope_fused;
  const uint16_t *qb, *kb, *vb;
  const float *bq, *bk, *bv;
  const float *inv_freq;
} aos_attn_params;

#define AOS_LAUNCH(ctx, kernel, grid, block, lds, ...)                                            \
  do {                                                                                            \
    if ((ctx)->ev_start)                                                                          \
      hipExtLaunchKernelGGL(kernel, grid, block, lds, (hipStream_t)(ctx)->stream,                 \
                            (hipEvent_t)(ctx)->ev_start, (hipEvent_t)(ctx)->ev_stop, 0, __VA_ARGS__); \
    else                                                                                          \
      hipLaunchKernelGGL(kernel, grid, block, lds, (hipStream_t)(ctx)->stream, __VA_ARGS__);      \
  } while (0)

/* A launcher with nothing to do still closes its profiling interval (zero length), so that
 * pooled events never report a stale time. */
#define AOS_SKIP(ctx)                                                                             \
  do {                                                                                            \
    if ((ctx)->ev_start) {                                                                        \
      (void)hipEventRecord((hipEvent_t)(ctx)->ev_start, (hipStream_t)(ctx)->stream);              \
      (void)hipEventRecord((hipEvent_t)(ctx)->ev_stop, (hipStream_t)(ctx)->stream);               \
    }                                                                                             \
  } while (0)

/* ---- Liquid blend: up to AOS_LIQUID_MAX adapters' deltas on one activation vector ----
 * down[a] = A [rank[a] x in], up[a] = B [up_rows[a] x rank[a]], row-major, float32 or bfloat16
 * (the *_bf16 flags); scaling[a] = alpha / rank. Entries past n have rank 0. */
#define AOS_LIQUID_MAX 3
#define AOS_LIQUID_RANK_MAX 1024
typedef struct {
  int n, in, out_len;
  const void *down[AOS_LIQUID_MAX], *up[AOS_LIQUID_MAX];
  int down_bf16[AOS_LIQUID_MAX], up_bf16[AOS_LIQUID_MAX];
  int rank[AOS_LIQUID_MAX], up_rows[AOS_LIQUID_MAX];
  float coef[AOS_LIQUID_MAX], scaling[AOS_LIQUID_MAX];
  const float *x; /* [in] */
  float *y;       /* [out_len] */
} aos_liquid_params;

#ifdef __cplusplus
extern "C" {
#endif
/* Host-side launchers (return hipError_t as int). */
int aos_launch_route(const aos_route_params *p, const aos_launch_ctx *ctx);
int aos_launch_embed(const aos_embed_params *p, const aos_launch_ctx *ctx);
int aos_launch_norm(const aos_norm_params *p, const aos_launch_ctx *ctx);
int aos_launch_rope(const aos_rope_params *p, const aos_launch_ctx *ctx);
int aos_launch_attention(const aos_attn_params *p, const aos_launch_ctx *ctx);
int aos_launch_shrink(const aos_shrink_params *p, const aos_launch_ctx *ctx);
int aos_launch_gemv(const aos_gemv_params *p, int swiglu, const aos_launch_ctx *ctx);
int aos_launch_gemv3(const aos_gemv3_params *p, const aos_launch_ctx *ctx);
int aos_launch_gemv_fused(const aos_gemv_fused_params *p, int swiglu, const aos_launch_ctx *ctx);
int aos_launch_decode_mlp(const aos_decode_mlp_params *p, const aos_launch_ctx *ctx);
/* consistency of a fused parameter block (sizes, generations, hand-off pointers) */
int aos_launch_liquid(const aos_liquid_params *p, const aos_launch_ctx *ctx);
int aos_fused_params_ok(const aos_gemv_fused_params *fp, int swiglu); /* 1: consistent */
int aos_launch_route_gate_up(const aos_route_gu_params *p, const aos_launch_ctx *ctx);
int aos_launch_gplan(const aos_gplan_params *p, const aos_launch_ctx *ctx);
int aos_launch_tshrink(const aos_tshrink_params *p, const aos_launch_ctx *ctx);
int aos_launch_amplan(const aos_amplan_params *p, const aos_launch_ctx *ctx);
int aos_launch_amshrink(const aos_amshrink_params *p, const aos_launch_ctx *ctx);
int aos_launch_amx(const aos_amx_params *p, const aos_launch_ctx *ctx);
int aos_launch_gemm(const aos_gemm_params *p, int swiglu, const aos_launch_ctx *ctx);
int aos_launch_xexp(const aos_xexp_params *p, const aos_launch_ctx *ctx);
int aos_gemm_shrink_fits(int T, int RB, int s_cols, int swiglu);
int aos_launch_mlp1(const aos_mlp1_params *p, const aos_launch_ctx *ctx);
/* The prefill GEMM's stream-K shape on the current device (swiglu: the gate/up kernel, else the
 * single-matrix one): workgroups resident at once, and floats of partial sums per workgroup. */
int aos_gemm_sk_slots(int swiglu);
int aos_gemm_sk_slot_floats(int swiglu);
int aos_spin_setter_mlp1(uint32_t polls);
/* The wait bound of each translation unit's kernels on the current device (polls; hipError_t). */
int aos_spin_setter_router(uint32_t polls);
int aos_spin_setter_lora(uint32_t polls);
int aos_spin_setter_gemv(uint32_t polls);
int aos_spin_setter_gemm(uint32_t polls);
int aos_spin_setter_model(uint32_t polls);
int aos_spin_setter_liquid(uint32_t polls);
#ifdef __cplusplus
}
#endif

#endif
