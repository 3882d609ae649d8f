/*
 * pallas_flash_amd.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * One entry point per launch site of the reference's Pallas operator layer
 * (aabhimittal/TPU-Native-Pallas-FlashAttention, src/pallas_flash). Each entry
 * point takes a plain-old-data argument struct (device pointers, sizes,
 * scalars) plus a HIP stream passed as `void*` (a hipStream_t; NULL = the
 * default stream), and returns a pf_status. No torch, XLA or HIP types appear
 * in the signatures.
 *
 * Conventions
 *  - Layout: every tensor is dense row-major (C-contiguous) in the shape given
 *    in the struct comments; element strides are implied by the shape.
 *  - Ownership: the caller allocates every buffer, including workspaces
 *    (pf_paged_attn_noalloc instead uses a static device array of the
 *    library's). Entry points never allocate, free or synchronise; they
 *    enqueue kernels on `stream` and return.
 *  - Validation happens on the host before any HIP call; a rejected call
 *    enqueues nothing. After enqueueing, hipGetLastError() is checked and a
 *    launch failure is reported as PF_ERR_LAUNCH.
 *  - Thread safety: reentrant. The only state is the process-wide tuning
 *    (pf_set_tuning), a per-device cache of the CU count and kernel
 *    occupancy (filled once per device under std::call_once), the per-device
 *    ticket counters of the prefill kernels' dynamic work tail (one per
 *    stream, assigned under a mutex; see pf_attn_fwd) and the per-device
 *    scratch array of pf_paged_attn_noalloc (see there).
 *  - Data types: dtype tags PF_DTYPE_F32 / PF_DTYPE_BF16 / PF_DTYPE_F16 name
 *    the storage type of q/k/v/o (and do/dq/dk/dv); all arithmetic is float32
 *    (MFMA with float32 accumulation). LSE / delta are always float32.
 *  - head_dim: 64, 128, or (bf16/f16) 256 for the prefill and RoPE entry
 *    points (a float32 tile of 256 columns would not fit the LDS double
 *    buffers); pf_attn_decode, pf_paged_attn, pf_paged_attn_noalloc and the
 *    cache writes take any head_dim up to 256 (bf16/f16) or 128 (float32)
 *    whose rows are whole 16-byte chunks (a multiple of 8 for bf16/f16, of 4
 *    for float32) and read or write the cache or pool rows in place. The
 *    reference bounds no head_dim; other values return PF_ERR_UNSUPPORTED.
 */
#ifndef PALLAS_FLASH_AMD_H
#define PALLAS_FLASH_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  PF_OK = 0,
  PF_ERR_INVALID = -1,      /* bad shape / pointer / scalar argument      */
  PF_ERR_UNSUPPORTED = -2,  /* valid but not implemented (dtype, head_dim) */
  PF_ERR_WORKSPACE = -3,    /* workspace missing or too small             */
  PF_ERR_LAUNCH = -4        /* HIP reported an error at launch            */
} pf_status;

typedef enum { PF_DTYPE_F32 = 0, PF_DTYPE_BF16 = 1, PF_DTYPE_F16 = 2 } pf_dtype;

/* ---------------------------------------------------------------------------
 * Forward prefill: o = softmax(scale * q k^T + mask) v, plus LSE.
 * Replaces the `flash_attention_fwd` pallas_call
 * (flash_attention.py:162-227, kernel :61-159).
 *   q   [batch, num_heads,    seq_len_q, head_dim]
 *   k,v [batch, num_kv_heads, seq_len_k, head_dim]
 *   o   [batch, num_heads,    seq_len_q, head_dim]   (same dtype as q)
 *   lse [batch, num_heads,    seq_len_q] float32, natural log of the scaled
 *       scores; may be NULL (not written). Rows with no valid key get o = 0,
 *       lse = 0.
 *   kv_len in (0, seq_len_k]; keys >= kv_len are never read.
 *   causal: q_pos >= k_pos, top-left aligned (also when seq_len_q != seq_len_k).
 * Work distribution: the kernel's work items (a query block of up to four
 * query heads of one GQA group) are placed on the GPU's XCDs in an L2-aware
 * order; with pf_tuning.tail_dynamic_pct > 0 and at least 1024 items, that
 * share of the items (the lightest) is instead handed out at run time to
 * whichever XCD is free, through a per-stream counter in a static device
 * array (no allocation; a launch recorded into a graph gets its own counter,
 * so two replays of one graph must not run at the same time -- replays of a
 * graph on one stream are ordered). Results are bit-identical either way.
 * Also applies to pf_attn_fwd_rope and to the dQ kernel of pf_attn_bwd_dq /
 * pf_attn_bwd (the dK/dV kernel places every item statically).
 * ------------------------------------------------------------------------- */
typedef struct {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int32_t batch, num_heads, num_kv_heads, seq_len_q, seq_len_k, head_dim;
  int32_t kv_len;
  int32_t causal;
  float sm_scale;
  int32_t dtype;
} pf_attn_fwd_args;

int pf_attn_fwd(const pf_attn_fwd_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Fused-RoPE forward (no LSE). Replaces the `flash_attention_rope_fwd`
 * pallas_call (fused_rope.py:183-213, kernel :53-113). Rotation is
 * x*cos + rotate_half(x)*sin in float32; for bf16/f16 the rotated Q and K are
 * rounded once to dtype before the matrix-core product (the reference keeps
 * them float32 for a float32 dot, fused_rope.py:75-78; float32 inputs stay
 * float32 here too). Q is rotated in registers inside the
 * attention kernel; K rows [0, kv_len) are rotated exactly once by a prologue
 * kernel into `workspace`, which the attention kernel then streams (the
 * reference re-rotates every K tile for every query head and query block).
 *   q_cos, q_sin [seq_len_q, head_dim] float32
 *   k_cos, k_sin [seq_len_k, head_dim] float32
 *   workspace: at least pf_attn_fwd_rope_workspace_size(args) bytes,
 *              256-byte aligned device memory (contents on entry do not matter)
 * Other fields as pf_attn_fwd_args (lse is ignored and may be NULL).
 * ------------------------------------------------------------------------- */
typedef struct {
  pf_attn_fwd_args base;
  const float* q_cos;
  const float* q_sin;
  const float* k_cos;
  const float* k_sin;
  void* workspace;
  size_t workspace_bytes;
} pf_attn_fwd_rope_args;

size_t pf_attn_fwd_rope_workspace_size(const pf_attn_fwd_rope_args* args);
int pf_attn_fwd_rope(const pf_attn_fwd_rope_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * RoPE rotation of a [batch, heads, seq_len, head_dim] tensor, the rotation
 * the fused forward applies (rotate-half, fused_rope.py:43-50; model.py:54-67).
 * With x1, x2 the two halves of a row and c1, c2, s1, s2 the halves of its
 * table rows:
 *   inverse = 0: out = x*cos + rotate_half(x)*sin
 *                (out1 = x1 c1 - x2 s1, out2 = x2 c2 + x1 s2)
 *   inverse = 1: the transpose of that linear map, i.e. its VJP -- the
 *                RoPE-aware backward (the reference's fused kernel is
 *                forward-only, README.md:156-157):
 *                out1 = x1 c1 + x2 s2, out2 = x2 c2 - x1 s1
 *                (exact for any table; for precompute_rope's tables, whose
 *                halves agree, it is x*cos - rotate_half(x)*sin)
 * Row s of every (batch, head) uses table row s; float32 arithmetic, one
 * rounding to dtype. x and out may alias.
 *   cos, sin [rope_len, head_dim] float32 with rope_len >= seq_len
 * ------------------------------------------------------------------------- */
typedef struct {
  const void* x;
  void* out;
  const float* cos;
  const float* sin;
  int32_t batch, heads, seq_len, head_dim, rope_len;
  int32_t inverse;
  int32_t dtype;
} pf_rope_args;

int pf_rope(const pf_rope_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Backward. Replaces `_flash_attention_bwd_call` (flash_attention.py:354-442):
 * the delta preprocess (:363-365), the `flash_attention_bwd_dq` pallas_call
 * (:379-398) and the `flash_attention_bwd_dkv` pallas_call plus the GQA group
 * sum (:403-436).
 *   q, o, do_, dq [batch, num_heads,    seq_len_q, head_dim]  (dtype)
 *   k, v, dk, dv  [batch, num_kv_heads, seq_len_k, head_dim]  (dtype)
 *   lse           [batch, num_heads, seq_len_q] float32 (from pf_attn_fwd)
 *   delta         [batch, num_heads, seq_len_q] float32 workspace, the
 *                 rowsum of o * do_: written by pf_attn_bwd_delta and (from
 *                 its own rows) by pf_attn_bwd_dq, read by pf_attn_bwd_dkv --
 *                 so dkv runs after either of the two; pf_attn_bwd runs dq,
 *                 then dkv.
 * dk/dv are summed over the num_heads/num_kv_heads query heads of each group in
 * float32 before the single cast to dtype. Keys >= kv_len get zero gradient.
 * ------------------------------------------------------------------------- */
typedef struct {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* do_;
  const float* lse;
  float* delta;
  void* dq;
  void* dk;
  void* dv;
  int32_t batch, num_heads, num_kv_heads, seq_len_q, seq_len_k, head_dim;
  int32_t kv_len;
  int32_t causal;
  float sm_scale;
  int32_t dtype;
} pf_attn_bwd_args;

int pf_attn_bwd_delta(const pf_attn_bwd_args* args, void* stream);
int pf_attn_bwd_dq(const pf_attn_bwd_args* args, void* stream);
int pf_attn_bwd_dkv(const pf_attn_bwd_args* args, void* stream);
/* dq (which also writes delta), then dkv, on one stream */
int pf_attn_bwd(const pf_attn_bwd_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Single-query decode against a contiguous KV cache. Replaces
 * `flash_attention_decode` (flash_attention.py:555-589), which the reference
 * runs as the forward pallas_call with block_q = 1 and kv_len = cache_len.
 * Split-KV: partial (m, l, acc) per KV chunk into `workspace`, then a combine.
 *   q [batch, num_heads, 1, head_dim]; o same shape
 *   k_cache, v_cache [batch, num_kv_heads, cache_size, head_dim]
 *   cache_len in (0, cache_size]; slots >= cache_len are never read.
 *   head_dim <= 256 (bf16/f16) or 128 (float32), a multiple of 8 (bf16/f16)
 *   or 4 (float32): rows are read in place; bf16/f16 with head_dim 128 run
 *   the streaming kernel, other head dims and float32 the generic kernel
 *   (computing at 64, 128 or 256 with the missing columns as zeros), with
 *   the same results to rounding.
 * workspace: at least pf_attn_decode_workspace_size(args) bytes, 256-byte
 * aligned device memory (contents on entry do not matter).
 * ------------------------------------------------------------------------- */
typedef struct {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  void* o;
  int32_t batch, num_heads, num_kv_heads, cache_size, head_dim;
  int32_t cache_len;
  float sm_scale;
  int32_t dtype;
  void* workspace;
  size_t workspace_bytes;
} pf_attn_decode_args;

size_t pf_attn_decode_workspace_size(const pf_attn_decode_args* args);
int pf_attn_decode(const pf_attn_decode_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Paged single-query attention. Replaces the `paged_flash_attention`
 * pallas_call (paged.py:151-192, kernel :45-99).
 *   q [batch, num_heads, 1, head_dim]; o same shape
 *   k_pages, v_pages [num_pages, num_kv_heads, page_size, head_dim]
 *   block_tables [batch, pages_per_seq] int32 (device): logical -> physical
 *   context_lens [batch] int32 (device): valid tokens per sequence.
 * Sequence b attends min(context_lens[b], pages_per_seq*page_size) tokens; a
 * non-positive length gives o = 0. Table entries at logical pages at or past
 * ceil(len / page_size) are never read (so -1 padding is legal); live entries
 * are clamped into [0, num_pages). Any page_size >= 1 is accepted (the
 * reference has no restriction). head_dim as pf_attn_decode. bf16/f16 with
 * head_dim 128 and page_size a multiple of 4 run the streaming kernel (each
 * 4-row load stays inside one page); other page sizes, dtypes and head dims
 * run the generic split-KV kernel, with the same results to rounding.
 * workspace: at least pf_paged_attn_workspace_size(args) bytes.
 * ------------------------------------------------------------------------- */
typedef struct {
  const void* q;
  const void* k_pages;
  const void* v_pages;
  const int32_t* block_tables;
  const int32_t* context_lens;
  void* o;
  int32_t batch, num_heads, num_kv_heads, num_pages, page_size, head_dim;
  int32_t pages_per_seq;
  float sm_scale;
  int32_t dtype;
  void* workspace;
  size_t workspace_bytes;
} pf_paged_attn_args;

size_t pf_paged_attn_workspace_size(const pf_paged_attn_args* args);
int pf_paged_attn(const pf_paged_attn_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Paged single-query attention that allocates nothing and takes no
 * workspace. No counterpart in the reference: it is for callers that cannot
 * allocate device memory -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc. Same arguments, kernels and results
 * as pf_paged_attn (bit for bit); `workspace` / `workspace_bytes` are
 * ignored. The split-KV partials go to a static device array of
 * PF_NOALLOC_SCRATCH_BYTES that each GPU the library runs on holds until the
 * process ends.
 *  - A call whose partials need more than PF_NOALLOC_SCRATCH_BYTES
 *    (pf_paged_attn_workspace_size(args) larger) returns PF_ERR_WORKSPACE
 *    and enqueues nothing. bf16/f16, head_dim 128, page_size % 4 == 0 (the
 *    streaming kernel) needs at most about 16.3 MiB at the default tuning on
 *    a 256-CU device, whatever the batch; the generic kernel needs about
 *    batch * num_heads * splits * 520 bytes.
 *  - A call uses the array of the device `stream` belongs to (the null
 *    stream's: the current device).
 *  - Every call on one GPU shares that GPU's array: calls that overlap on
 *    one GPU (different streams, or other host threads) race on it and must
 *    be serialised by the caller. Nothing carries over between calls.
 *  - The array's device address is resolved once per device
 *    (hipGetSymbolAddress, with that device current) at the first call on it,
 *    also when that call is being recorded into a graph (the lookup runs
 *    with the thread's capture mode relaxed); no call allocates or frees.
 * ------------------------------------------------------------------------- */
#define PF_NOALLOC_SCRATCH_BYTES (32u << 20)
int pf_paged_attn_noalloc(const pf_paged_attn_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * KV-cache writes on device. Replaces the decode loop's `_cache_write`
 * (model.py:257-262, called at :299, :342, :487) and the ring-buffer slot
 * scatter of prefill_ring (model.py:437, :447-448) / ring_decode_step
 * (:475-476): rows [0, seq_len) of k/v go to slots pos + i of the contiguous
 * cache (ring = 0), or to slots (pos + i) mod cache_size (ring = 1; only the
 * last cache_size rows are written, so no two rows target one slot, which
 * keeps the tail prefill_ring keeps).
 *   k, v            [batch, num_kv_heads, seq_len, head_dim]     (dtype)
 *   k_cache, v_cache [batch, num_kv_heads, cache_size, head_dim] (dtype)
 *   positions       device int32: absolute position of row 0, read at
 *                   b * positions_stride (stride 0: one position for all).
 * A row whose slot is out of range (linear: pos + i outside [0, cache_size);
 * ring: pos + i < 0) is not written (the reference's dynamic_update_slice
 * would clamp it onto a valid slot instead). head_dim as pf_attn_decode.
 * ------------------------------------------------------------------------- */
typedef struct {
  const void* k;
  const void* v;
  void* k_cache;
  void* v_cache;
  const int32_t* positions;
  int32_t positions_stride;
  int32_t batch, num_kv_heads, seq_len, cache_size, head_dim;
  int32_t ring;
  int32_t dtype;
} pf_kv_cache_write_args;

int pf_kv_cache_write(const pf_kv_cache_write_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Paged-pool write (batched). Replaces `write_to_paged_cache`
 * (paged.py:205-223), which writes one token of one sequence: row i of
 * sequence b lands at position p = positions[b * positions_stride] + i, i.e.
 * physical page block_tables[b][p / page_size], offset p % page_size.
 *   k, v              [batch, num_kv_heads, seq_len, head_dim]          (dtype)
 *   k_pages, v_pages  [num_pages, num_kv_heads, page_size, head_dim]    (dtype)
 *   block_tables      [batch, pages_per_seq] int32 (device)
 * A row is not written when p < 0, its logical page is >= pages_per_seq, or
 * its table entry lies outside [0, num_pages) (e.g. -1 padding). Rows of
 * different sequences that map to one (page, offset) race; the caller keeps
 * them distinct (pages shared between sequences are for read-only prefixes).
 * head_dim as pf_attn_decode.
 * ------------------------------------------------------------------------- */
typedef struct {
  const void* k;
  const void* v;
  void* k_pages;
  void* v_pages;
  const int32_t* block_tables;
  const int32_t* positions;
  int32_t positions_stride;
  int32_t batch, num_kv_heads, seq_len, num_pages, page_size, head_dim, pages_per_seq;
  int32_t dtype;
} pf_paged_cache_write_args;

int pf_paged_cache_write(const pf_paged_cache_write_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Fused decode step. Replaces the attention part of one decode_step /
 * ring_decode_step layer (model.py:340-347, :485-491): RoPE of the new
 * token's q and k at its position (rotate-half, float32, rounded once), the
 * cache write of k and v at its slot, and single-query attention over the
 * live slots. Positions live in device memory and no host-side value depends
 * on them, so one captured step (HIP graph) replays as the caller advances
 * them on the GPU -- the reference instead re-traces per step because
 * kv_len is static (flash_attention.py:448).
 *   q      [batch, num_heads, 1, head_dim]     pre-RoPE (dtype)
 *   k_new, v_new [batch, num_kv_heads, 1, head_dim]  k pre-RoPE (dtype)
 *   k_cache, v_cache [batch, num_kv_heads, cache_size, head_dim]
 *   o      [batch, num_heads, 1, head_dim]
 *   positions  device int32, read at b * positions_stride
 *   cos, sin   [rope_len, head_dim] float32 (precompute_rope), or both NULL
 *              for no rotation
 *   ring = 0: slot pos, attends slots [0, pos] (valid iff 0 <= pos < cache_size)
 *   ring = 1: slot pos % cache_size, attends min(pos + 1, cache_size) slots
 *             (valid iff pos >= 0); model.py:475-476
 * With RoPE, a valid position is also < rope_len. An invalid position writes
 * nothing and gives o = 0 for that batch.
 * Supported: bf16 / f16 with head_dim 128 (PF_ERR_UNSUPPORTED otherwise).
 * workspace: at least pf_attn_decode_step_workspace_size(args) bytes,
 * 256-byte aligned (contents on entry do not matter).
 * ------------------------------------------------------------------------- */
typedef struct {
  const void* q;
  const void* k_new;
  const void* v_new;
  void* k_cache;
  void* v_cache;
  void* o;
  const int32_t* positions;
  int32_t positions_stride;
  const float* cos;
  const float* sin;
  int32_t rope_len;
  int32_t batch, num_heads, num_kv_heads, cache_size, head_dim;
  int32_t ring;
  float sm_scale;
  int32_t dtype;
  void* workspace;
  size_t workspace_bytes;
} pf_attn_decode_step_args;

size_t pf_attn_decode_step_workspace_size(const pf_attn_decode_step_args* args);
int pf_attn_decode_step(const pf_attn_decode_step_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Process-wide tuning of kernel variants and launch shapes. Every setting
 * computes the same attention (to float rounding order). No counterpart in
 * the reference, whose only tuning inputs are the static block_q / block_k
 * arguments of its pallas_calls (flash_attention.py:479-490), which this
 * build accepts and ignores. Initial values come from the environment, read
 * once per process at the first launch or tuning call:
 *   PF_TAIL_DYNAMIC_PCT   0 .. 100 (default 30): percentage of the forward's
 *                         and dQ's work items (the lightest) handed out at run
 *                         time to whichever XCD is free (0: every item placed
 *                         statically; see pf_attn_fwd)
 *   PF_DECODE_STAGES      2 (default) .. 4: LDS ring depth of the streaming
 *                         decode / paged kernel
 *   PF_DECODE_WAVES       0 (default: one per resident slot, queried once per
 *                         device) or the persistent decode grid size
 * pf_set_tuning replaces all three for later calls (PF_ERR_INVALID for values
 * outside those ranges; launches already enqueued are unaffected). Safe to
 * call from any thread.
 * ------------------------------------------------------------------------- */
typedef struct {
  int32_t tail_dynamic_pct;
  int32_t decode_stages;
  int32_t decode_waves;
} pf_tuning;

int pf_get_tuning(pf_tuning* out);
int pf_set_tuning(const pf_tuning* tuning);

/* Library version string (static storage). */
const char* pf_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PALLAS_FLASH_AMD_H */
