/*
 * treeattn.h -- C ABI of the MI355X (gfx950) segment-tree sparse attention library (libtreeattn.so).
 *
 * The reference (Dex8123/treeattn) has no native code: its hot path is PyTorch ops plus three Triton
 * kernels reached from Python.  Each entry point below replaces one reference function or op chain,
 * cited as file:line of the reference.  The Python package treeattn_amd binds these through ctypes and
 * keeps the reference's Python signatures on top.
 *
 * Conventions (all entry points):
 *   - Device pointers, explicit sizes and element strides, a hipStream_t passed as void*.  Work is
 *     enqueued on that stream; nothing is synchronised and nothing is allocated.  Scratch memory, where
 *     needed, is a caller-provided workspace whose size a *_workspace_size() function reports.
 *   - Tensors of rows are addressed as base + b*sb + h*sh + n*sn with the last (feature) dimension
 *     contiguous; strides are in elements.
 *   - Element types: TA_F32, TA_F16, TA_BF16.  Index tensors are int32, -1 meaning "no entry".
 *   - Return 0 on success, a TA_ERR_* code otherwise; ta_last_error() gives a message (per thread).
 *   - Node sums ("pyramid") are float32.  Tree level j (j = 0 is the leaf-block level) holds nodes of
 *     leaf * arity^j positions; node m covers [m*size, (m+1)*size).  Level j is passed as a device base
 *     pointer plus its batch and head strides; node rows are contiguous with stride D.
 */
#ifndef TREEATTN_H_
#define TREEATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TA_ABI_VERSION 3

enum ta_dtype { TA_F32 = 0, TA_F16 = 1, TA_BF16 = 2 };

enum ta_status {
  TA_OK = 0,
  TA_ERR_ARG = 1,       /* bad size, stride, alignment or dtype */
  TA_ERR_UNSUPPORTED = 2, /* shape outside what the kernels are built for */
  TA_ERR_LAUNCH = 3,    /* the HIP runtime refused the launch */
  TA_ERR_WORKSPACE = 4  /* workspace too small */
};

int ta_abi_version(void);
const char* ta_last_error(void);

/* 1 when the current HIP device is a gfx950 the library has code for, 0 otherwise. */
int ta_device_supported(void);

/*
 * Paged decode cache (replaces the contiguous per-layer K/V of engine.py:26-27, SegState; no counterpart for
 * the layout itself in the reference).  A page holds the rows of one leaf block of one (sequence, head): with
 * pages, row r (r < 2^block_log2) of leaf block j of (b, h) lives at
 *   K: Kc + table[b*sb + h*sh + j] * page_stride + r * cst,   V: Vc + (same page) * page_stride + r * cst,
 * so Kc / Vc are the bases of page 0's K and V rows and the per-sequence and per-head cache strides are not
 * used.  A page id outside [0, num_pages) means "no page": such rows are never read and never written.
 * Entry points taking `const ta_kv_pages* pages` use the contiguous layout when it is NULL.
 */
typedef struct ta_kv_pages {
  const int32_t* table;   /* device memory, int32 page ids */
  int64_t sb, sh;         /* element strides of the table for sequence and head */
  int64_t page_stride;    /* elements from one page to the next (K and V alike) */
  int64_t num_pages;
  int block_log2;         /* rows per page = 2^block_log2 = the leaf block of the tree */
} ta_kv_pages;

/*
 * The neighbour store of the selection (engine.py:103-105) that a descent can write as it writes its outputs:
 * for a query at position t in [0, Tst) and slot r < n, leaf[b,h,t,r] = the r-th kept leaf id (0 past the kept
 * ones), score = its score (0 past them), ok = 1 for a kept leaf else 0.  leaf int32 / score float32 / ok uint8
 * (B, H, Tst, >= n) share the element strides sb, sh, st; n <= wl.
 */
typedef struct ta_leaf_store_out {
  int32_t* leaf;
  float* score;
  uint8_t* ok;
  int64_t sb, sh, st;
  int Tst;
  int n;
} ta_leaf_store_out;

/*
 * Level-sum pyramid of a key tensor (replaces seg.py:26-41 level_sums, fastseg.py:238-251 level_sums_min
 * without the gate, and the index-key preparation seg.py:128-130 / fastseg.py:306-308).
 *
 * k: (B, H, T, D) of k_dtype.  Index keys are k as float32, with position 0 zeroed when zero_sink is 1
 * (seg.py:130; level_sums itself sums whatever it is given, seg.py:31-35).  Every node of the
 * binary levels 1.. is the sum of its two children (children added left + right, in float32), and the
 * levels listed in lv_* are written: lv_blevel[j] is the binary level (log2 of the node size) of output
 * level j, strictly increasing.  Only nodes lying completely inside [0, t_end) are written.
 * ws: float32 workspace of ta_level_sums_workspace_size(...) bytes.
 */
int64_t ta_level_sums_workspace_size(int B, int H, int t_end, int D);
int ta_level_sums(const void* k, int k_dtype, int64_t ksb, int64_t ksh, int64_t kst,
                  int B, int H, int t_end, int D, int zero_sink,
                  int n_levels, float* const* lv_ptr, const int64_t* lv_sb, const int64_t* lv_sh,
                  const int32_t* lv_blevel,
                  float* ws, int64_t ws_bytes, void* stream);

/*
 * Beam descent with per-query top-k leaf-block selection (replaces seg.py:44-70 tree_pass and
 * fastseg.py:254-271 tree_pass_fast, including the per-level gather_dot of fastseg.py:267 and topk).
 *
 * q: (B, H, Nq, D) of q_dtype (scored in float32).  tq: query positions, tq[b*tq_sb + n] (tq_sb = 0 to
 * share one position list across the batch).  The tree spans [0, T) (T a power of two) with leaf blocks
 * of 2^leaf_log2 keys and 2^arity_log2 children per node; the n_levels pyramid levels are tree levels
 * 0..n_levels-1 in ta_level_sums layout.
 * Semantics: at every level, top first, the candidates are the children of the kept nodes plus the
 * complete left siblings of the node containing t; a node's score is q . sum / size in the canonical
 * float32 order (per-dimension products without fused multiply-add, 16 groups of D/16 consecutive
 * dimensions each reduced by the halving tree, then the halving tree over the 16 group sums, times the
 * exact power of two 1/size); the best wmax by (score desc, node id asc) are kept.
 * Outputs (B, H, Nq, wl) contiguous: ids (leaf-block ids, best first; -1 past the valid ones), vld (0/1),
 * sct (scores; -inf past the valid ones).  wl is the reference's leaf beam width for this geometry.
 * A query whose position lies outside [0, T) selects nothing.
 */
int ta_tree_descend(const void* q, int q_dtype, int64_t qsb, int64_t qsh, int64_t qsn,
                    int B, int H, int Nq, int D,
                    const int32_t* tq, int64_t tq_sb,
                    int n_levels, const float* const* lv_ptr, const int64_t* lv_sb, const int64_t* lv_sh,
                    int T, int leaf_log2, int arity_log2, int wmax, int wl,
                    int32_t* ids, uint8_t* vld, float* sct, void* stream);

/* ta_tree_descend that also writes each query's neighbour store (store non-NULL; engine.py:103-105). */
int ta_tree_descend_store(const void* q, int q_dtype, int64_t qsb, int64_t qsh, int64_t qsn,
                          int B, int H, int Nq, int D,
                          const int32_t* tq, int64_t tq_sb,
                          int n_levels, const float* const* lv_ptr, const int64_t* lv_sb, const int64_t* lv_sh,
                          int T, int leaf_log2, int arity_log2, int wmax, int wl,
                          int32_t* ids, uint8_t* vld, float* sct, const ta_leaf_store_out* store, void* stream);

/*
 * One decode position per (sequence, head): ta_tree_descend of q (B,H,1,D) at t = t_pos[b], and, in the same
 * launch, ta_kv_append of k_new / v_new at row t_pos[b] (the selection and cache update of one decode step,
 * engine.py:96-105 then engine.py:41-55).  The descent reads only nodes that end before t and the append
 * writes row t and the nodes ending at t, so the results equal the two calls made one after the other.
 * q, k_new, v_new and the caches share dtype; B*H < 4096; the levels are written (the append's nodes).
 */
int ta_tree_descend_append(const void* q, int dtype, int64_t qsb, int64_t qsh, int B, int H, int D,
                           const int32_t* t_pos, int n_levels, float* const* lv_ptr, const int64_t* lv_sb,
                           const int64_t* lv_sh, int T, int leaf_log2, int arity_log2, int wmax, int wl,
                           int32_t* ids, uint8_t* vld, float* sct,
                           const void* k_new, const void* v_new, int64_t nsb, int64_t nsh, int64_t vnsb,
                           int64_t vnsh, void* Kc, void* Vc, int64_t csb, int64_t csh, int64_t cst, int Tcap,
                           const ta_kv_pages* pages, void* stream);

/*
 * ta_tree_descend_append with two options: app_lv_ptr / app_lv_sb / app_lv_sh (n_levels entries, or NULL) name the
 * levels the append forms its nodes in when they are not the scored ones (the mean-log gate: gated levels are
 * scored from their gated vectors while the append forms the raw sums; the gate's own node update follows as
 * ta_gate_append), and store (or NULL) the position's neighbour store (engine.py:103-105), as
 * ta_tree_descend_store writes it.  gate_lg (n_levels log-sum levels, or NULL) with gate_out (gated-vector levels,
 * NULL entries where a level is not gated, or NULL) and gate_q: the same launch then does ta_gate_append's work for
 * the nodes the append completes (the levels sharing the append levels' strides; D <= 128).
 */
int ta_tree_descend_append_ex(const void* q, int dtype, int64_t qsb, int64_t qsh, int B, int H, int D,
                              const int32_t* t_pos, int n_levels, float* const* lv_ptr, const int64_t* lv_sb,
                              const int64_t* lv_sh, int T, int leaf_log2, int arity_log2, int wmax, int wl,
                              int32_t* ids, uint8_t* vld, float* sct,
                              const void* k_new, const void* v_new, int64_t nsb, int64_t nsh, int64_t vnsb,
                              int64_t vnsh, void* Kc, void* Vc, int64_t csb, int64_t csh, int64_t cst, int Tcap,
                              const ta_kv_pages* pages, float* const* app_lv_ptr, const int64_t* app_lv_sb,
                              const int64_t* app_lv_sh, float* const* gate_lg, float* const* gate_out,
                              float gate_q, const ta_leaf_store_out* store, void* stream);

/*
 * Scores of queries against gathered rows (replaces fastseg.py:118-130 gather_dot and its kernel
 * fastseg.py:34-47).  out[b,h,n,c] = scale * q[b,h,n] . S[b,h,clamp(cand[b,h,n,c], 0, M-1)], float32,
 * canonical order.  q: (B,H,N,D) q_dtype; S: (B,H,M,D) s_dtype; cand: (B,H,N,C) int32 contiguous;
 * out: (B,H,N,C) float32 contiguous.
 */
int ta_gather_dot(const void* q, int q_dtype, int64_t qsb, int64_t qsh, int64_t qsn,
                  const void* S, int s_dtype, int64_t ssb, int64_t ssh, int64_t ssn,
                  const int32_t* cand, int B, int H, int N, int M, int C, int D, float scale,
                  float* out, void* stream);

/*
 * Leaf-block gather-dot: the candidates of a query are whole blocks of `block` consecutive rows,
 * out[b,h,n, c*block + j] = scale * q[b,h,n] . K[b,h, blk[b,h,n,c]*block + j] (fastseg.py:118-130 with
 * cand = blk*block + arange(block)).  blk: (B,H,N,NB) int32 contiguous, ids in [0, M/block); as in the
 * reference every key position is clamped into [0, M) (fastseg.py:121), so an id below 0 scores row 0 for all
 * its keys and an id at or past M/block row M - 1.  Same dtype for q and K; out (B,H,N,NB*block) float32 contiguous.
 * For bf16/f16 with D in {64, 128}, block in {32, 64, 128}, M a multiple of block, NB <= 64 and 16-byte
 * aligned rows, the scores come from matrix-core products of the exact bf16/f16 values with float32
 * accumulation (a few ulps from a sequential float32 sum); other shapes use the canonical order of
 * ta_gather_dot.
 */
int ta_gather_dot_blocks(const void* q, const void* K, int dtype,
                         int64_t qsb, int64_t qsh, int64_t qsn, int64_t ksb, int64_t ksh, int64_t ksn,
                         const int32_t* blk, int B, int H, int N, int M, int NB, int block, int D,
                         float scale, float* out, void* stream);

/*
 * Candidate list of the module forward, masked (replaces fastseg.py:367-381 and attention_dyn.py:74-86: the
 * concatenation of tree, neighbour and static keys, their validity, and dedupe_fast / attention_dyn.py:12-17,
 * the first valid copy of each position).  Per query row (B,H,N): tree_pos (leaf * wl positions, entry r * wl
 * + j = position r of found leaf j, -1 = none), leaf_ok (wl bytes), n_tree (leaves to use), nb_pos (nbk
 * positions), all int64 / uint8 and contiguous; tq: the rows' positions, (N) or (B,N) when tq_batched, int64.
 * The candidates are tree_pos, nb_pos, then 0, t, t-1, ..., t-Lw+1 (Lw = max(local, 3); negatives -1) and, for
 * leaf > 2, the query's own leaf group up to t; KC = leaf * wl + nbk + 1 + Lw (+ leaf), at most 320.  cm:
 * (B,H,N,KC) int32, the position where kept, else -1 (what ta_sparse_attn_fwd takes); counts: (B,H,N,4) int32:
 * kept entries, kept tree entries, kept neighbour entries, leaves used (found and within n_tree).
 */
int ta_assemble_candidates(const int64_t* tree_pos, const uint8_t* leaf_ok, const int64_t* n_tree,
                           const int64_t* nb_pos, const int64_t* tq, int tq_batched, int B, int H, int N, int wl,
                           int leaf, int nbk, int local, int32_t* cm, int32_t* counts, void* stream);

/*
 * Softmax attention of each query over an explicit candidate list (replaces fastseg.py:173-177
 * sparse_attn forward, its kernel fastseg.py:50-78 and the fallback fastseg.py:134-141).
 * q: (B,H,T,D), k, v: (B,H,Tk,D), same dtype; cand: (B,H,T,KC) int32 contiguous, -1 = unused, duplicates
 * counted as given; positions >= Tk are treated as unused.  out: (B,H,T,D) contiguous in the input dtype; lse: (B,H,T)
 * float32 (may be NULL).  Softmax in float32; a row with no valid candidate gives out = 0, lse = -1e30.
 */
int ta_sparse_attn_fwd(const void* q, const void* k, const void* v, int dtype,
                       int64_t qsb, int64_t qsh, int64_t qst, int64_t ksb, int64_t ksh, int64_t kst,
                       int64_t vsb, int64_t vsh, int64_t vst,
                       const int32_t* cand, int B, int H, int T, int Tk, int KC, int D, float scale,
                       void* out, float* lse, const ta_kv_pages* pages, void* stream);

/*
 * Backward of ta_sparse_attn_fwd (replaces fastseg.py:81-110 _attn_bwd and fastseg.py:158-170
 * _SparseAttnFn.backward): given q, k, v, the forward's out o and lse, and dout = dL/do, with
 * p_j = exp(scale q.k_j - lse) over the valid slots, Dq = dout . o and ds_j = p_j (dout . v_j - Dq):
 *   dq = scale sum_j ds_j k_j  (written, input dtype, (B,H,T,D) contiguous),
 *   dk[cand_j] += scale ds_j q,  dv[cand_j] += p_j dout  (float32 (B,H,Tk,D) contiguous).
 * Slots as in the forward (-1 or >= Tk unused, duplicates counted).  q, o, dout: element strides (b, h, t)
 * with the last dimension contiguous; k, v rows 16-byte aligned.  D a multiple of 8 up to 256, B*H <= 65535.
 * dq is deterministic.  dk and dv:
 *   ws non-NULL (ta_sparse_attn_bwd_workspace_size bytes): written (every key row, zeros where no slot names
 *     it), each key's contributions added in a fixed order (queries ascending, slots ascending) -- bit for bit
 *     reproducible.  causal: every candidate position is at most its query's position (T == Tk), which lets a
 *     key skip the queries before it.
 *   ws NULL: accumulated into with float32 atomic adds, as the reference's kernel does (zero them first); the
 *     summation order then depends on scheduling (reproducible to float32 rounding).
 */
int ta_sparse_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout, int dtype,
                       int64_t qsb, int64_t qsh, int64_t qst, int64_t ksb, int64_t ksh, int64_t kst,
                       int64_t vsb, int64_t vsh, int64_t vst, int64_t osb, int64_t osh, int64_t ost,
                       int64_t dsb, int64_t dsh, int64_t dst, const int32_t* cand, const float* lse,
                       int B, int H, int T, int Tk, int KC, int D, float scale, void* dq, float* dk, float* dv,
                       float* ws, int causal, void* stream);

/* Bytes of the deterministic route's workspace of ta_sparse_attn_bwd (per-slot ds and p, float32). */
int64_t ta_sparse_attn_bwd_workspace_size(int B, int H, int T, int KC);

/*
 * Attention over the keys a descent selected (replaces fastseg.py:367-383 candidate assembly +
 * dedupe_fast + sparse_attn, and engine.py:107-119 for one decode position), neighbours off.
 * The key set of query n (position t = tq[b*tq_sb + n]) is the union of
 *   - the first min(n_tree[b,h,n], #valid) leaf blocks of ids/vld (n_tree NULL: all valid ones),
 *   - the query's own partial leaf block [leaf*floor(t/leaf), t],
 *   - the static keys {0, t, t-1, ..., t-Lw+1} (>= 0), Lw = max(local, 3),
 * each position once.  q: (B,H,Nq,D) with strides; k, v: (B,H,Tk,D) with strides (the whole sequence or a
 * KV cache); positions outside [0, Tk) are never read (a query with t >= Tk attends nothing).  ids/vld: (B,H,Nq,wl) contiguous.  out: (B,H,Nq,D) in the input dtype with strides; lse:
 * (B,H,Nq) float32 or NULL; keys: (B,H,Nq) float32 number of keys attended, or NULL.
 * nsplit is 1 (one wavefront per query) or a multiple of 4 up to 256: the keys of every query are split
 * over nsplit wavefronts (for few queries with many keys, as in decode), 4 per workgroup merged in LDS; with
 * more than 4, nsplit/4 workgroups per query write partials to ws (ta_seg_attn_workspace_size(...) bytes,
 * 256-byte aligned, zero-filled once when allocated: its head holds per-query counters that every call
 * leaves at zero) and the last workgroup of each query merges them.  Calls that share a workspace must not
 * run concurrently.
 */
int64_t ta_seg_attn_workspace_size(int B, int H, int Nq, int D, int nsplit);
int ta_seg_attn_fwd(const void* q, const void* k, const void* v, int dtype,
                    int64_t qsb, int64_t qsh, int64_t qsn, int64_t ksb, int64_t ksh, int64_t kst,
                    int64_t vsb, int64_t vsh, int64_t vst,
                    int B, int H, int Nq, int D, int Tk,
                    const int32_t* tq, int64_t tq_sb,
                    const int32_t* ids, const uint8_t* vld, const int32_t* n_tree, int wl,
                    int leaf, int local, float scale,
                    void* out, int64_t osb, int64_t osh, int64_t osn, float* lse, float* keys,
                    int nsplit, float* ws, int64_t ws_bytes, const ta_kv_pages* pages, void* stream);

/*
 * ta_seg_attn_fwd in the reference-default selection mode (neighbour borrowing on; replaces the candidate
 * assembly and first-copy dedupe of fastseg.py:367-383 / engine.py:107-114 and the attention over the
 * result): besides the first n_tree valid tree leaves, each query attends the leaf blocks of its matched
 * neighbour slots -- nb_id / nb_ok (B, H, Nq, nb_S) int32 / uint8, query qi's slots at qi * nb_S, as
 * ta_neighbor_pass writes them -- each block once (a block already among the tree leaves, or held by an
 * earlier matched slot, or not complete before the query's own block, is skipped), then the own block and the
 * static keys outside every attended block.  nb_S <= 64.  keys[qi] counts the keys of that set.  Otherwise as
 * ta_seg_attn_fwd (the vector kernels serve every shape here).
 */
int ta_seg_attn_nb_fwd(const void* q, const void* k, const void* v, int dtype,
                       int64_t qsb, int64_t qsh, int64_t qsn, int64_t ksb, int64_t ksh, int64_t kst,
                       int64_t vsb, int64_t vsh, int64_t vst,
                       int B, int H, int Nq, int D, int Tk,
                       const int32_t* tq, int64_t tq_sb,
                       const int32_t* ids, const uint8_t* vld, const int32_t* n_tree, int wl,
                       int leaf, int local, float scale, const int32_t* nb_id, const uint8_t* nb_ok, int nb_S,
                       void* out, int64_t osb, int64_t osh, int64_t osn, float* lse, float* keys,
                       int nsplit, float* ws, int64_t ws_bytes, const ta_kv_pages* pages, void* stream);

/*
 * ta_seg_attn_fwd without a workspace argument: no counterpart in the reference (it has no workspaces).  For
 * callers that cannot allocate device memory -- code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc.  The split attention's scratch (ta_seg_attn_workspace_size(...) bytes: per-query
 * counters and per-workgroup partials) lives in a fixed array of TA_SCRATCH_BYTES bytes that the library holds
 * on every GPU it runs on until the process ends; a call needing more returns TA_ERR_WORKSPACE (use
 * ta_seg_attn_fwd with a workspace then).  The call allocates nothing.  Every call on one GPU shares that GPU's
 * array: calls that overlap in time on one GPU race and must be ordered (one stream).  Arguments and results as
 * ta_seg_attn_fwd, bit for bit.
 */
#define TA_SCRATCH_BYTES (4 << 20)
int ta_seg_attn_fwd_noalloc(const void* q, const void* k, const void* v, int dtype,
                            int64_t qsb, int64_t qsh, int64_t qsn, int64_t ksb, int64_t ksh, int64_t kst,
                            int64_t vsb, int64_t vsh, int64_t vst,
                            int B, int H, int Nq, int D, int Tk,
                            const int32_t* tq, int64_t tq_sb,
                            const int32_t* ids, const uint8_t* vld, const int32_t* n_tree, int wl,
                            int leaf, int local, float scale,
                            void* out, int64_t osb, int64_t osh, int64_t osn, float* lse, float* keys,
                            int nsplit, const ta_kv_pages* pages, void* stream);

/*
 * One decode step of one layer's attention in one launch (replaces seg_attend in the structural mode,
 * engine.py:84-120, with SegState.add, engine.py:41-55): per (sequence, head), the cache append of
 * k_new / v_new at row t = t_pos[b] (and the nodes it completes), the beam descent of q (B,H,1,D) at t, and the
 * attention over the kept leaf blocks (the first min(n_tree[b,h], kept) of them), the own block and the static
 * keys, one workgroup per (sequence, head).  The selection is written to ids / vld / sct (B,H,1,wl) as
 * ta_tree_descend writes it; out (B,H,1,D) strides osb, osh; keys (B,H,1) float32 or NULL.  Equals
 * ta_tree_descend_append followed by ta_seg_attn_fwd with nsplit 4, bit for bit.  D is 64 or 128, wl <= 64;
 * q, new rows, caches and output share dtype; the levels are written (the append's nodes).
 */
int ta_seg_attend(const void* q, const void* k_new, const void* v_new, int dtype, int64_t qsb, int64_t qsh,
                  int64_t nsb, int64_t nsh, int64_t vnsb, int64_t vnsh, int B, int H, int D,
                  const int32_t* t_pos, int n_levels, float* const* lv_ptr, const int64_t* lv_sb,
                  const int64_t* lv_sh, int T, int leaf_log2, int arity_log2, int wmax, int wl,
                  void* Kc, void* Vc, int64_t csb, int64_t csh, int64_t cst, int Tcap,
                  const int32_t* n_tree, int local, float scale,
                  int32_t* ids, uint8_t* vld, float* sct, void* out, int64_t osb, int64_t osh, float* keys,
                  const ta_kv_pages* pages, void* stream);

/*
 * Decode-cache append with incremental node formation (replaces engine.py:41-55 SegState.add and the
 * state writes of engine.py:102-106).  For every sequence b at position t = t_pos[b]: row t of the K and
 * V caches (B,H,Tcap,D, cache dtype) takes k_new, v_new (B,H,D with strides, same dtype as the cache);
 * then every pyramid node whose last position is t is formed: a leaf block as the adjacent-pair sum of
 * its keys (position 0 counted as 0), a higher node as the adjacent-pair sum of its children.
 */
int ta_kv_append(const void* k_new, const void* v_new, int dtype,
                 int64_t nsb, int64_t nsh, int64_t vnsb, int64_t vnsh,
                 void* Kc, void* Vc, int64_t csb, int64_t csh, int64_t cst,
                 int B, int H, int D, int Tcap, const int32_t* t_pos,
                 int n_levels, float* const* lv_ptr, const int64_t* lv_sb, const int64_t* lv_sh,
                 int leaf_log2, int arity_log2, const ta_kv_pages* pages, void* stream);

/*
 * Row-block matrix product of the decode step (the model around the attention: model.py:21-44,
 * engine.py:168-177 -- F.linear with the LayerNorm before it and GELU / residual add after it), bf16:
 *   Y[M,N] = epilogue( LN(X)[M,K] . W[N,K]^T ),  LN applied when ln_w != NULL (no bias, eps ln_eps),
 *   epilogue 0: none, 1: GELU (erf), 2: residual add R + (.).  Each op's result is rounded to bf16 as in
 * the unfused chain.  Row strides ldx, ldw, ldy, ldr in elements; K a multiple of 64; X, W, ln_w 16-byte
 * aligned.  Y may be the same buffer as R.
 * splits > 1 divides K among that many workgroups per 32 x 32 output tile (clamped to K/64); their float32
 * partials are summed in split order, so results are deterministic.
 * Tails, done once by the last output tile to finish (at most one per call):
 *   ln_next != NULL: y_ln[M, N] = LN(Y) with weight ln_next (eps ln_eps) -- the LayerNorm the next product
 *     of the residual stream applies (model.py:42-44, LN1 / LN2 / LN_f), bit for bit the prologue's
 *     arithmetic; N a multiple of 64, Y, y_ln and ln_next 16-byte aligned (row stride ld_yln);
 *   tok_out != NULL: tok_out[m] = the first column of the largest bf16 value of row m of Y (the greedy
 *     token of the reference's loop, phase2.py:51-66; NaN never chosen, 0 for a row of NaN); no epilogue.
 * ws: ta_rowmm_workspace_size bytes, 256-byte aligned, zero-filled once when allocated (its counters and
 * keys return to zero after every call), needed when splits > 1 or a tail is asked for.  Calls that share a
 * workspace must not overlap in time.
 */
int64_t ta_rowmm_workspace_size(int M, int N, int K, int splits);
int ta_rowmm(const void* X, int64_t ldx, const void* W, int64_t ldw, void* Y, int64_t ldy,
             const void* R, int64_t ldr, const void* ln_w, float ln_eps, int M, int N, int K,
             int epilogue, int splits, const void* ln_next, void* y_ln, int64_t ld_yln, int64_t* tok_out,
             void* ws, int64_t ws_bytes, void* stream);

/*
 * ta_rowmm with the output tile chosen by the caller: cols = 4, 8, 16 or 32 columns per workgroup of eight
 * wavefronts (one per K-block stream, operands loaded straight into registers), -1 for the four-wavefront
 * 32-column tile with X staged in LDS, 0 for the library's choice (what ta_rowmm does: the widest of 32/16/8
 * columns that still gives every compute unit a workgroup).  Every choice computes the same bits: the same
 * K-block streams, MFMA chains and stream-order sums (an MFMA output column depends only on its own column of
 * W).  The tails (ln_next, tok_out) always run on the 32-column tile.
 */
int ta_rowmm_ex(const void* X, int64_t ldx, const void* W, int64_t ldw, void* Y, int64_t ldy,
                const void* R, int64_t ldr, const void* ln_w, float ln_eps, int M, int N, int K,
                int epilogue, int splits, int cols, const void* ln_next, void* y_ln, int64_t ld_yln,
                int64_t* tok_out, void* ws, int64_t ws_bytes, void* stream);

/*
 * Logits of a decode step and their greedy token (replaces engine.py:177, F.linear(ln_f(x), wte), and
 * logits.argmax(-1) of the reference's greedy loop, phase2.py:51-66), bf16, for up to 32 rows:
 *   Y[M,N] = LN(X)[M,K] . W[N,K]^T  (LN applied when ln_w != NULL, eps ln_eps), bit for bit ta_rowmm's
 *   result with epilogue 0;  tok_out[m] (when tok_out != NULL) = the first column of the largest bf16 value
 *   of row m of Y (NaN never chosen, 0 for a row of NaN), as ta_argmax_rows.
 * 1 <= M <= 32, K a multiple of 64 up to 1024; X, W, ln_w 16-byte aligned with 16-byte row strides.  Each
 * workgroup normalises the rows once and walks several 32-column tiles (the next tile's W in flight while one
 * is multiplied); the last workgroup to finish reduces the per-workgroup row maxima.
 * ws (needed with tok_out): ta_logits_workspace_size bytes, 256-byte aligned, zero-filled once when
 * allocated (its counter returns to zero after every call); calls sharing a workspace must not overlap.
 */
int64_t ta_logits_workspace_size(int M, int N);
int ta_logits(const void* X, int64_t ldx, const void* W, int64_t ldw, void* Y, int64_t ldy, const void* ln_w,
              float ln_eps, int M, int N, int K, int64_t* tok_out, void* ws, int64_t ws_bytes, void* stream);

/*
 * The float32 decode step's row products for a few rows (replaces engine.py:168-177 at float32: F.linear(ln_1(x),
 * c_attn), x + F.linear(y, c_proj), F.gelu(F.linear(ln_2(x), c_fc)), x + F.linear(h, c_mlp), F.linear(ln_f(x),
 * wte)), one launch each:
 *   Y[M,N] = epilogue(LN(X)[M,K] . W[N,K]^T), LN applied when ln_w != NULL (eps ln_eps, no bias), epilogue 0
 *   none, 1 exact GELU, 2 + R[M,N] (R may be Y).
 * 1 <= M <= 8, K <= 2048, float32, rows contiguous with strides ldx, ldw, ldy, ldr (elements); X must not
 * overlap Y.  Float32 sums in the kernel's order (within float32 rounding of the framework's products).
 */
int ta_rowvec_f32(const float* X, int64_t ldx, const float* W, int64_t ldw, float* Y, int64_t ldy, const float* R,
                  int64_t ldr, const float* ln_w, float ln_eps, int M, int N, int K, int epilogue, void* stream);

/*
 * ta_rowmm's row product (LayerNorm prologue, product, epilogue; replaces the same engine.py:168-177 products at
 * bf16) for one to eight rows without matrix cores: one wavefront per output column, the same arithmetic at
 * every rounding point (float32 LayerNorm statistics from the sums of x and x^2, the normalised row rounded to
 * bf16, float32 products summed in float32, the sum rounded to bf16 before GELU or the residual); only the
 * order of the float32 sums differs, so outputs agree with ta_rowmm's within one bf16 unit.  What the bf16
 * decoder runs for one or two rows, where a matrix-core tile computes mostly idle rows.
 * 1 <= M <= 8, K a multiple of 8 up to 4096; X, W, ln_w 16-byte aligned, row strides multiples of 8 elements;
 * X must not overlap Y (R may be Y).
 */
int ta_rowvec_bf16(const void* X, int64_t ldx, const void* W, int64_t ldw, void* Y, int64_t ldy, const void* R,
                   int64_t ldr, const void* ln_w, float ln_eps, int M, int N, int K, int epilogue, void* stream);

/*
 * Row-wise argmax for greedy decoding (replaces logits.argmax(-1) of the reference's greedy loop,
 * phase2.py:51-66): out[r] = the first index of the largest value of x[r, 0:n].  x: rows of n elements of
 * dtype with row stride `stride`; out: int64.
 */
int ta_argmax_rows(const void* x, int dtype, int64_t rows, int64_t n, int64_t stride, int64_t* out,
                   void* stream);

/*
 * First op of a decode step (engine.py:168, x = wte[tok] + wpe[t]): x[b, :] = wte[tok[b], :] + wpe[t[b], :]
 * in dtype (the sum rounded once), pos32[b] = t[b]; with `advance`, t[b] += 1 afterwards (the next step's
 * position, so a captured step can be replayed).  tok, t: int64 (B,); tables with row strides ldw, ldp.
 * ln_w != NULL (bf16, C a multiple of 64, at most 4096): also x_ln[b, :] = LN(x[b, :]) with weight ln_w and
 * eps ln_eps, the first layer's LN1 (model.py:43), bit for bit as ta_rowmm computes it.
 */
int ta_embed(const int64_t* tok, int64_t* tpos, int advance, const void* wte, int64_t ldw, const void* wpe,
             int64_t ldp, int dtype, int B, int C, int64_t V, int64_t P, void* x, int64_t ldx, int32_t* pos32,
             const void* ln_w, float ln_eps, void* x_ln, int64_t ld_xln, void* stream);

/*
 * float32 -> bf16 with the rounding every kernel of the library uses (round to nearest even; NaN stays NaN):
 * out[i] = bf16(in[i]), bit patterns.  in 16-byte and out 8-byte aligned.  (Lets a test hold the kernels'
 * rounding against the reference framework's.)
 */
int ta_bf16_from_f32(const float* in, uint16_t* out, int64_t n, void* stream);

/*
 * The whole decode step in one launch (replaces Decoder.step, engine.py:161-177, with seg_attend in the
 * structural mode, engine.py:84-120, SegState.add, engine.py:41-55, and the greedy argmax of
 * phase2.py:51-66): embedding, every layer (LN1 + c_attn, cache append + beam descent + attention per
 * (sequence, head), c_proj + residual, LN2 + c_fc + GELU, c_mlp + residual), LN_f + logits and the greedy
 * token, for a bf16 GPT with head_dim 64 and up to 32 sequences.  The results equal the per-op entry
 * points above run in the same order (ta_rowmm with the same split of c_mlp, ta_tree_descend_append,
 * ta_seg_attn_fwd with one workgroup per query, ta_argmax_rows), bit for bit.
 *
 * ta_decode_step_prepare writes the step's plan (task list, tensor addresses) into the workspace `ws`
 * (ta_decode_step_workspace_size bytes, 256-byte aligned; it also holds the step's activations and
 * counters), zeroes its counters, waits for the stream, and fills `out` with the launch shape.  The model's
 * tensors must stay at the addresses given.  ta_decode_step then enqueues one step: tokens tok (B, int64)
 * at positions tpos (B, int64) -> logits (B, vocab) bf16 with row stride ld_logits; tok_out (may alias
 * tok, or NULL) receives the greedy tokens; with `advance` every tpos[b] is incremented; keys (n_layer,
 * B, n_head) float32, or NULL, receives the keys attended; trace (launch->n_tasks, 16) int64, or NULL,
 * receives per task the wall-clock ticks (hipDeviceAttributeWallClockRate) when a workgroup took it, when
 * its input wait ended, at up to ten points inside it (0 where a task has none) and when it finished, then
 * that workgroup's CU id and two zeros.  Steps that share a workspace must not overlap
 * in time.  The step waits on its own counters with a bounded wait (two seconds); when one runs out the
 * step completes with wrong results and ta_decode_step_error reports 1 (it reads the flag synchronously;
 * the flag stays set until the next prepare).
 */
#define TA_MAX_TREE_LEVELS 32

typedef struct ta_step_layer {
  const void* ln1;       /* (n_embd) */
  const void* c_attn;    /* (3 n_embd, n_embd) */
  const void* c_proj;    /* (n_embd, n_embd) */
  const void* ln2;       /* (n_embd) */
  const void* c_fc;      /* (n_ff, n_embd) */
  const void* c_mlp;     /* (n_embd, n_ff) */
  void* k_cache;         /* (batch, n_head, tcap, head_dim) */
  void* v_cache;         /* same shape and strides as k_cache */
  int64_t c_sb, c_sh, c_st;
  float* levels[TA_MAX_TREE_LEVELS];   /* node sums of tree level j (node rows of head_dim floats) */
  int64_t lv_sb[TA_MAX_TREE_LEVELS], lv_sh[TA_MAX_TREE_LEVELS];
} ta_step_layer;

typedef struct ta_step_model {
  int n_layer, n_head, head_dim, n_embd, n_ff, vocab, n_pos, batch, tcap;
  int leaf, arity, n_levels, wmax, n_tree, local;
  int mlp_splits;        /* workgroups per c_mlp output tile along K */
  float ln_eps;
  const void* wte;       /* (vocab, n_embd), row stride ld_wte; also the tied output head */
  int64_t ld_wte;
  const void* wpe;       /* (n_pos, n_embd), row stride ld_wpe */
  int64_t ld_wpe;
  const void* ln_f;      /* (n_embd) */
  const ta_step_layer* layers;   /* n_layer entries (host memory) */
} ta_step_model;

typedef struct ta_step_launch {
  int grid, lds_bytes, n_tasks, head_dim;
} ta_step_launch;

int64_t ta_decode_step_workspace_size(const ta_step_model* m);
int ta_decode_step_prepare(const ta_step_model* m, void* ws, int64_t ws_bytes, ta_step_launch* out, void* stream);
int ta_decode_step(const ta_step_launch* launch, void* ws, const int64_t* tok, int64_t* tok_out, int64_t* tpos,
                   int advance, void* logits, int64_t ld_logits, float* keys, int64_t* trace, void* stream);
int ta_decode_step_error(const void* ws, int* error, void* stream);

/*
 * Neighbour borrowing (replaces seg.py:73-103 neighbor_pass and fastseg.py:274-299 neighbor_pass_fast, and with
 * lhat the budget split of seg.py:111-117).  For every query n of (b, h) at position t = tq[b * tq_sb + n]: the
 * S = nb_window * nb_store stored slots of positions t - 1 .. t - nb_window (slot s: position t - (s / nb_store
 * + 1), entry s % nb_store of st_*), each stored leaf scored against q with the canonical float32 dot times
 * scale (the gather-dot's order; ids clamped into [0, M)); match = valid and score >= base - nb_rho * |base|;
 * rate = matches / max(valid, 1) over the first nb_probe * nb_store slots; a slot of neighbour back is kept
 * when back <= nb_cap_min + round_half_even((nb_window - nb_cap_min) * rate); none when neighbors == 0.
 * Outputs: nid (B, H, Nq, S) int32 the stored leaf ids (0 for an empty slot), match (uint8), nL (B, H, Nq)
 * distinct matched leaves, and with lhat (budgets, int32 (B, H, Nq)) n_tree = 0 if nL >= L else max(L - nL,
 * 2 if nL < ceil(L / 2) else 1), at most wmax.
 * q: (B, H, Nq, D) of q_dtype, D 16, 32, 64, 128 or 256; S0: the leaf-level node sums (B, H, M, D) float32 (batch and head
 * strides ssb, ssh); st_leaf int32 / st_score float32 / st_ok uint8 (B, H, Tst, nb_store) with element strides
 * st_sb, st_sh, st_st; S <= 64.
 */
int ta_neighbor_pass(const void* q, int q_dtype, int64_t qsb, int64_t qsh, int64_t qsn, const float* S0,
                     int64_t ssb, int64_t ssh, int M, const int32_t* st_leaf, const float* st_score,
                     const uint8_t* st_ok, int64_t st_sb, int64_t st_sh, int64_t st_st, int Tst,
                     const int32_t* tq, int64_t tq_sb, int B, int H, int Nq, int D, int nb_window,
                     int nb_store, int nb_probe, int nb_cap_min, float nb_rho, int neighbors, float scale,
                     const int32_t* lhat, int wmax, int32_t* nid, uint8_t* match, int32_t* nL,
                     int32_t* n_tree, void* stream);

/*
 * The decode step's budget head (replaces the feature / linear / argmax sequence of engine.py:89-96) for every
 * (b, h): features f = [q (D), log(|q| + 1e-6), one-hot(h) (H)] plus, when ksum is given, ksum[b,h] / max(t_pos[b],
 * 1) (D); lhat[b*H + h] = classes[argmax(W2 relu(W1 f + b1) + b2)], float32 throughout, the first maximum winning.
 * q (B, H, D) rows of q_dtype at element strides qsb, qsh; ksum float32 (B, H, D) contiguous or null; with k (same
 * dtype as q, strides ksb, ksh) the key sum then takes this step's key (ksum += k).  w1t is W1 transposed,
 * float32 (F, hid) row-major with F = D + 1 + H (+ D with ksum); w2 float32 (ncls, hid); hid <= 256,
 * ncls <= 64, 2 D + 1 + H <= 1024, (F + ncls) * hid <= 24576.
 */
int ta_budget_head(const void* q, int q_dtype, int64_t qsb, int64_t qsh, float* ksum, const void* k, int64_t ksb,
                   int64_t ksh, const int32_t* t_pos, const float* w1t, const float* b1, const float* w2,
                   const float* b2, const int32_t* classes, int B, int H, int D, int hid, int ncls, int32_t* lhat,
                   void* stream);

/*
 * The budget head of a decode step as ta_neighbor_pass_head takes it (the weights as ta_budget_head takes them:
 * W1 transposed (F x hid) and W2 (ncls x hid) float32, 16-byte aligned, hid a multiple of 4 and <= 256,
 * ncls <= 64; ksum (B, H, D) float32 contiguous or NULL without the global pool; k this step's keys (q's dtype,
 * strides ksb, ksh) added to ksum after its read, or NULL; lhat (B, H) int32 receives the budgets, or NULL).
 */
typedef struct ta_budget_head_in {
  const float* w1t;
  const float* b1;
  const float* w2;
  const float* b2;
  const int32_t* classes;
  int hid, ncls;
  float* ksum;
  const void* k;
  int64_t ksb, ksh;
  int32_t* lhat;
} ta_budget_head_in;

/*
 * One decode position per (sequence, head): ta_budget_head and ta_neighbor_pass with its budget split in one
 * launch (engine.py:89-102).  q (B, H, D) rows at strides qsb, qsh; t_pos (B,) positions; the other arguments as
 * ta_neighbor_pass's with Nq = 1; n_tree receives the split of the head's budget.  The budgets and the key sum
 * equal ta_budget_head's, bit for bit.
 */
int ta_neighbor_pass_head(const void* q, int q_dtype, int64_t qsb, int64_t qsh, const float* S0, int64_t ssb,
                          int64_t ssh, int M, const int32_t* st_leaf, const float* st_score, const uint8_t* st_ok,
                          int64_t st_sb, int64_t st_sh, int64_t st_st, int Tst, const int32_t* t_pos, int B, int H,
                          int D, int nb_window, int nb_store, int nb_probe, int nb_cap_min, float nb_rho,
                          int neighbors, float scale, int wmax, const ta_budget_head_in* head, int32_t* nid,
                          uint8_t* match, int32_t* nL, int32_t* n_tree, void* stream);

/*
 * The decode step's neighbour store (replaces the assignments of engine.py:103-105): for every (b, h) and slot
 * r < n, at position t = t_pos[b] (skipped outside [0, Tst)): st_leaf[b,h,t,r] = ids[b,h,0,r] (an invalid slot's
 * -1 stored as 0), st_score = sct when vld else 0, st_ok = vld.  ids int32 / vld uint8 / sct float32 are the
 * descent's (B, H, 1, wl) contiguous outputs; st_leaf int32 / st_score float32 / st_ok uint8 (B, H, Tst, nb_store)
 * share the element strides st_sb, st_sh, st_st; n <= wl.
 */
int ta_leaf_store(const int32_t* ids, const uint8_t* vld, const float* sct, int B, int H, int wl, int n,
                  const int32_t* t_pos, int32_t* st_leaf, float* st_score, uint8_t* st_ok, int64_t st_sb,
                  int64_t st_sh, int64_t st_st, int Tst, void* stream);

/*
 * Log-magnitude pyramid for the mean-log gate (seg.py:33, 39; engine.py:47, 53-54): ta_level_sums over the
 * values log(|x| + 1e-6) of the index keys x (position 0 counted as 0 when zero_sink) instead of the keys --
 * each log the float32 rounding of the double-precision log of the float32 |x| + 1e-6 -- with the same
 * adjacent-pair float32 additions.  Arguments as ta_level_sums (same workspace size).
 */
int ta_level_log_sums(const void* k, int k_dtype, int64_t ksb, int64_t ksh, int64_t kst,
                      int B, int H, int t_end, int D, int zero_sink,
                      int n_levels, float* const* lv_ptr, const int64_t* lv_sb, const int64_t* lv_sh,
                      const int32_t* lv_blevel, float* ws, int64_t ws_bytes, void* stream);

/*
 * Mean-log gate of node summaries (replaces seg.py:16-23 gate_apply as applied by seg.py:37-38, fastseg.py:
 * 248-249 and SegState.getU, engine.py:35-39).  For level j (binary level blevel[j], nodes of 2^blevel
 * positions) and every node n < n_nodes[j] of every (b, h): ml = lg / 2^blevel per dimension; thr = the gate_q
 * quantile of ml over the D dimensions (order statistics at floor and ceil of r = gate_q * (D - 1) in float32,
 * interpolated as torch.lerp: lo + w (hi - lo) for w < 0.5, else hi - (hi - lo)(1 - w), w = r - floor(r), each
 * operation rounded); out = (raw * [ml >= thr]) * (D / max(#kept, 1)).  raw, lg, out: (B, H, M_j, D) float32
 * with node rows contiguous and batch / head strides sb[j], sh[j]; out[j] == NULL skips level j.  D 16 to 128.
 */
int ta_gate_levels(int B, int H, int D, int n_levels, const float* const* raw, const float* const* lg,
                   float* const* out, const int64_t* sb, const int64_t* sh, const int32_t* blevel,
                   const int64_t* n_nodes, float gate_q, void* stream);

/*
 * The gate's share of a decode-cache append (engine.py:47, 53-54), after ta_kv_append has written row t_pos[b]
 * and the raw nodes ending at it: forms the log-magnitude sums of the nodes ending at t (the leaf block's index
 * keys read back from the K cache Kc -- contiguous (B, H, Tcap, D) with strides csb, csh, cst, or pages -- then
 * every completed parent from its children, as the raw sums are formed) and the gated vectors of those nodes
 * on levels whose out[j] is not NULL, as ta_gate_levels computes them.  Levels are tree levels 0.. with
 * blevel[0] = log2(leaf) and arity 2^arity_log2; lg is written, raw read.
 */
int ta_gate_append(const void* Kc, int dtype, int64_t csb, int64_t csh, int64_t cst, int Tcap, int B, int H, int D,
                   const int32_t* t_pos, int n_levels, const float* const* raw, float* const* lg,
                   float* const* out, const int64_t* sb, const int64_t* sh, const int32_t* blevel,
                   int arity_log2, float gate_q, const ta_kv_pages* pages, void* stream);

/*
 * Calibration (no counterpart in the reference): wgs workgroups of four wavefronts each run 4 * iters
 * v_mfma_f32_32x32x16_bf16 instructions (32768 flops each) on register operands, no memory traffic; timing the
 * launch gives the dense bf16 matrix-core throughput the GPU sustains, the peak a kernel's MFMA utilisation is
 * set against.  out: wgs floats (written only in a case that does not occur; it keeps the work alive).
 */
int ta_mfma_peak(int wgs, int iters, float* out, void* stream);

/*
 * Block forest (the reference's attn='block' attention), step 1 -- replaces forest.py:47-75 build_forest with
 * forest.py:12-33 two_means_order and forest.py:36-44 soft_gate.  Keys k (B, H, T, D), D 16, 32, 64 or 128 (row 0,
 * the sink, counted as zero), cut into blocks of `block` keys (a power of two in [4, 64] dividing T; depth = log2(block / 2)):
 * every block's keys are ordered by depth rounds of 2-means splits of its groups (kmeans_iters iterations each),
 * perm (B, H, T) int32 gets rank -> position inside the block, and sums[l] (B, H, (T / block) << l, D) float32
 * (l = 0..depth; strides sb[l], sh[l], node rows contiguous) the node sums of every level (level 0 = the block,
 * level depth = pairs of ranks; flat node id = block index * 2^l + m).  With gate, the soft gate (quantile
 * gate_q, temperature gate_temp) is applied to every node sum in place; lg[l] (same layout) is its scratch.
 */
int ta_forest_build(const void* k, int dtype, int64_t ksb, int64_t ksh, int64_t kst, int B, int H, int T, int D,
                    int block, int kmeans_iters, int gate, float gate_q, float gate_temp, int32_t* perm,
                    float* const* sums, float* const* lg, const int64_t* sb, const int64_t* sh, void* stream);

/*
 * Block forest, step 2 -- replaces attention.py:88-148 (the descent over the block trees, the budget's cut,
 * leaves to key positions, static keys and their duplicates).  For every query t of q (B, H, T, D): the roots of
 * all blocks are scored (q . node sum; valid: the blocks before t's own), the best min(wmax, C) kept (valid while
 * their rank is below bq_desc), their two children scored, ... down to the pairs.  Writes leaf / leafv
 * (B, H, T, wl) and cand (B, H, T, Kc) int32: [own block positions (the causal ones) | 0, t-1, t-2 (inside
 * earlier blocks) | the two keys of every used leaf, all first keys then all second keys], -1 where unused; a
 * leaf is used when valid and its rank is below bq_use[b, h, t] (bq_use NULL: every valid leaf); a key equal to
 * a valid static key is dropped.  lv_cur / lv_cv (NULL or (depth + 1, B, H, T, lv_stride)): every level's
 * candidates and their validity (-1 / 0 past the level's count), for the routing loss.  counts (NULL or
 * (B, H, T, 2) int32): each row's valid static keys and tree keys (the counts behind attention.py:135-137's
 * statistics, from the kernel that writes the row).  wl, Kc and the widest level: ta_forest_shape.
 */
int ta_forest_descend(const void* q, int dtype, int64_t qsb, int64_t qsh, int64_t qst, int B, int H, int T, int D,
                      int block, const float* const* sums, const int64_t* sb, const int64_t* sh,
                      const int32_t* perm, int wmax, int bq_desc, const int32_t* bq_use, int32_t* leaf,
                      uint8_t* leafv, int32_t* cand, int32_t* lv_cur, uint8_t* lv_cv, int lv_stride,
                      int32_t* counts, void* stream);

/* Leaves per query (wl), candidate-list width (Kc = block + 3 + 2 wl) and widest level of ta_forest_descend. */
int ta_forest_shape(int T, int block, int wmax, int* wl, int* kc, int* widest);

/*
 * LaneTree (the reference's attn='dyn' selection), workspace -- bytes of the lane trees of ta_lanetree_build /
 * ta_lanetree_walk: B * H * (T / chunk) trees of capacity T, each T * (4 D + 8) bytes (node sums float32, counts
 * and leaf slots int32).  T a power of two in [4, 262144], chunk dividing T, D 16, 32, 64 or 128.  Above
 * T = 16384 the build and the walk keep the leaf slots in this workspace rather than in LDS, and the build's sort
 * entries in a tree's node-sum area until it writes the node sums (the results are the same).
 */
int ta_lanetree_workspace_size(int B, int H, int T, int D, int chunk, int64_t* bytes);

/*
 * LaneTree, step 1 -- replaces dyntree.py:34-82 LaneTree.__init__ with dyntree.py:6-31 masked_two_means_order,
 * for every lane of dyntree.py:161-166: lane l of every (b, h) gets a tree of capacity T over the keys
 * [1, l * chunk) of k (B, H, T, D): log2(T) - 1 rounds of masked 2-means splits (kmeans_iters iterations each),
 * every group's real keys laid out half and half, then the node sums and counts.  ws: the workspace above.
 */
int ta_lanetree_build(const void* k, int dtype, int64_t ksb, int64_t ksh, int64_t kst, int B, int H, int T, int D,
                      int chunk, int kmeans_iters, void* ws, int64_t ws_bytes, void* stream);

/*
 * LaneTree, step 2 -- replaces dyntree.py:148-243 select_keys (with dyntree.py:84-131 insert / search /
 * leaf_keys) on the trees of ta_lanetree_build, which it updates.  Every lane walks its positions t in order:
 * the neighbour test over the leaves the lane's last nb_window positions stored (nb_store each; score >=
 * base - nb_rho |base|, the cap from the match rate of the first nb_probe positions), the leaf budget from
 * lhat (B, H, T) int32, the beam search (node score q . mean key, wmax wide), then the insertion of key t.
 * Writes tree_pos (B, H, T, 2 wl) int32 [all first keys | all second keys] of the found leaves (wl =
 * min(wmax, T / 2)), leaf_ok (B, H, T, wl), nb_pos (B, H, T, 2 nb_window nb_store) int32, n_tree and nb_leaves
 * (B, H, T) int32, -1 / 0 where unused.  1 <= wmax <= 64, nb_window * nb_store <= 64, nb_store <= wl.
 */
int ta_lanetree_walk(const void* q, const void* k, int dtype, int64_t qsb, int64_t qsh, int64_t qst, int64_t ksb,
                     int64_t ksh, int64_t kst, int B, int H, int T, int D, int chunk, const int32_t* lhat, int wmax,
                     int nb_window, int nb_store, float nb_rho, int nb_probe, int nb_cap_min, int neighbors,
                     void* ws, int64_t ws_bytes, int32_t* tree_pos, uint8_t* leaf_ok, int32_t* nb_pos,
                     int32_t* n_tree, int32_t* nb_leaves, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TREEATTN_H_ */
