// extern "C" entry points of libpallas_flash_amd.so (declared in
// include/pallas_flash_amd.h). Each one validates its arguments on the host
// (no HIP call before validation passes), fills a kernel parameter block and
// enqueues on the caller's stream. Nothing here allocates or synchronises.
#include <math.h>
#include <stdlib.h>

#include <atomic>
#include <mutex>

#include "../../include/pallas_flash_amd.h"
#include "pf_kernels.hpp"

namespace {

// Process-wide tuning (pf_get_tuning / pf_set_tuning). The environment is read
// once, at the first call that needs a value; afterwards every launch reads
// three atomics and makes no environment or device query of its own.
// Share of a prefill launch's work items handed out by tickets (plan_tail).
constexpr int kDefaultTailDynamicPct = 30;

struct Tuning {
  std::atomic<int> tail_dynamic_pct{kDefaultTailDynamicPct};
  std::atomic<int> decode_stages{2};
  std::atomic<int> decode_waves{0};
};

bool tuning_valid(int dyn, int stages, int waves) {
  return dyn >= 0 && dyn <= 100 && stages >= 2 && stages <= 4 && waves >= 0;
}

Tuning& tuning() {
  static Tuning t;
  static std::once_flag once;
  std::call_once(once, [] {
    const char* f = getenv("PF_TAIL_DYNAMIC_PCT");
    const char* s = getenv("PF_DECODE_STAGES");
    const char* w = getenv("PF_DECODE_WAVES");
    if (f != nullptr && atoi(f) >= 0 && atoi(f) <= 100) t.tail_dynamic_pct = atoi(f);
    if (s != nullptr && atoi(s) >= 2 && atoi(s) <= 4) t.decode_stages = atoi(s);
    if (w != nullptr && atoi(w) > 0) t.decode_waves = atoi(w);
  });
  return t;
}

bool dtype_ok(int32_t d) { return d == PF_DTYPE_F32 || d == PF_DTYPE_BF16 || d == PF_DTYPE_F16; }
// Kernel head dims: 64 and 128 for every dtype, 256 for bf16/f16 (a float32
// tile of 256 columns would not fit the LDS double buffers). dtype must
// already be valid.
int32_t max_head_dim(int32_t dtype) { return dtype == PF_DTYPE_F32 ? 128 : 256; }
bool head_dim_ok(int32_t d, int32_t dtype) { return d == 64 || d == 128 || (d == 256 && d <= max_head_dim(dtype)); }

// Decode and paged decode also read rows of any head_dim up to the dtype's
// maximum that are whole 16-byte chunks (a multiple of 8 elements for
// bf16/f16, 4 for float32) in place: the generic kernel computes at the next
// kernel head dim with the missing columns as zeros.
bool decode_head_dim_ok(int32_t d, int32_t dtype) {
  const int32_t es = dtype == PF_DTYPE_F32 ? 4 : 2;
  return d >= 1 && d <= max_head_dim(dtype) && (d * es) % 16 == 0;
}
int32_t decode_compute_dim(int32_t d) { return d <= 64 ? 64 : d <= 128 ? 128 : 256; }

constexpr int64_t kMaxGrid = 0x7fffffff;

int check_attn_dims(int32_t B, int32_t Hq, int32_t Hkv, int32_t Sq, int32_t Sk, int32_t D,
                    int32_t kv_len, float scale, int32_t dtype) {
  // flash_attention.py:527-545: ranks/shape agreement, Hq % Hkv, kv_len in (0, Sk].
  if (B < 0 || Hq < 1 || Hkv < 1 || Sq < 0 || Sk < 1 || D < 1) return PF_ERR_INVALID;
  if (Hq % Hkv != 0) return PF_ERR_INVALID;
  if (kv_len < 1 || kv_len > Sk) return PF_ERR_INVALID;
  if (!isfinite(scale)) return PF_ERR_INVALID;
  if (!dtype_ok(dtype)) return PF_ERR_UNSUPPORTED;
  if (!head_dim_ok(D, dtype)) return PF_ERR_UNSUPPORTED;
  return PF_OK;
}

int finish(hipError_t e) { return e == hipSuccess ? PF_OK : PF_ERR_LAUNCH; }

// (batch, kv head) pairs each XCD streams at a time in the forward
// (fwd_work_item): with more than one pair per XCD, the largest divisor of
// the per-XCD pair count whose pairs' live K/V (kv_len rows each) fits an
// XCD's 4 MB L2, at least 1; 0 (the default item order) when the pairs are
// not a multiple of the 8 XCDs or one pair per XCD. (Config 2's shape, four
// 2 MiB pairs per XCD: two at a time measured 1.5% faster than one and as
// fast as all four, with half of their HBM traffic.)
int fwd_pair_group(const pf_attn_fwd_args* a) {
  const int64_t npairs = (int64_t)a->batch * a->num_kv_heads;
  if (npairs % 8 != 0 || npairs == 8) return 0;
  const int per_xcd = (int)(npairs / 8);
  const int64_t es = a->dtype == PF_DTYPE_F32 ? 4 : 2;
  const int64_t pair_bytes = (int64_t)a->kv_len * a->head_dim * es * 2;
  int best = 1;
  for (int P = 1; P <= per_xcd; ++P)
    if (per_xcd % P == 0 && P * pair_bytes <= (int64_t)(4 << 20)) best = P;
  return best;
}

int fill_fwd(const pf_attn_fwd_args* a, pf::FwdParams* p) {
  int st = check_attn_dims(a->batch, a->num_heads, a->num_kv_heads, a->seq_len_q, a->seq_len_k,
                           a->head_dim, a->kv_len, a->sm_scale, a->dtype);
  if (st != PF_OK) return st;
  if (!a->q || !a->k || !a->v || !a->o) return PF_ERR_INVALID;
  p->q = a->q;
  p->k = a->k;
  p->v = a->v;
  p->o = a->o;
  p->lse = a->lse;
  p->q_cos = p->q_sin = nullptr;
  p->B = a->batch;
  p->Hq = a->num_heads;
  p->Hkv = a->num_kv_heads;
  p->Sq = a->seq_len_q;
  p->Sk = a->seq_len_k;
  p->kv_len = a->kv_len;
  p->g = a->num_heads / a->num_kv_heads;
  p->scale_log2 = a->sm_scale * 1.4426950408889634f;
  // A workgroup's 4 waves cover hpw query heads of one GQA group x rpw rows:
  // the K/V tiles it stages serve all of them.
  p->hpw = (p->g % 4 == 0) ? 4 : (p->g % 2 == 0) ? 2 : 1;
  p->rpw = 128 / p->hpw;
  p->n_qblk = (a->seq_len_q + p->rpw - 1) / p->rpw;
  const int64_t n_work = (int64_t)a->batch * (a->num_heads / p->hpw) * p->n_qblk;
  if (n_work > kMaxGrid) return PF_ERR_UNSUPPORTED;
  // per-(batch, kv head) byte offsets are 32-bit inside the kernels
  if ((int64_t)(a->seq_len_k + 256) * a->head_dim * 4 > 0x7fffffff) return PF_ERR_UNSUPPORTED;
  p->n_work = (int)n_work;
  p->pair_group = fwd_pair_group(a);
  p->tail = pf::WorkTail{nullptr, p->n_work, 0};
  return PF_OK;
}

// Dynamic tail of a prefill launch (pf::WorkTail): the last tail_dynamic_pct
// percent of the work items (the lightest under the heavy-first orders) go to
// ticket-drawing workgroups, kTailSlack times as many as those items so an
// XCD that runs ahead can take up to that multiple of its share. The static
// part is a multiple of the 8 XCDs so each gets the same number of its own
// items. Launches of fewer than min_items items (two per resident workgroup
// slot of the kernel) keep every item static, as do launches whose stream
// gets no ticket counter. The dK/dV kernel, one workgroup per CU and two
// items per CU, gains nothing from a tail (measured) and runs without one:
// its items drawn by other XCDs only add HBM traffic (889 against 578 MB at
// config 3).
constexpr double kTailSlack = 2.0;

pf::WorkTail plan_tail(int n_work, int min_items, hipStream_t stream) {
  pf::WorkTail w{nullptr, n_work, 0};
  const int pct = tuning().tail_dynamic_pct.load(std::memory_order_relaxed);
  if (pct <= 0 || n_work < min_items) return w;
  const int n_static = 8 * (int)(((int64_t)n_work * (100 - pct) / 100) / 8);
  const int pool = n_work - n_static;
  if (pool <= 0) return w;
  unsigned int* t = pf::work_tickets(stream);
  if (t == nullptr) return w;
  w.tickets = t;
  w.n_static = n_static;
  w.n_tickets = (int)(pool * kTailSlack) + 1;
  return w;
}

// Minimum items for a dynamic tail: two per resident workgroup slot of a
// 256-CU MI355X (the 16-bit forward and dQ run two workgroups per CU).
constexpr int kTwoPerCu = 2 * 2 * 256;

}  // namespace

extern "C" {

const char* pf_version(void) { return "pallas_flash_amd 0.1.0 (gfx950)"; }

int pf_get_tuning(pf_tuning* out) {
  if (!out) return PF_ERR_INVALID;
  Tuning& t = tuning();
  out->tail_dynamic_pct = t.tail_dynamic_pct.load();
  out->decode_stages = t.decode_stages.load();
  out->decode_waves = t.decode_waves.load();
  return PF_OK;
}

int pf_set_tuning(const pf_tuning* in) {
  if (!in || !tuning_valid(in->tail_dynamic_pct, in->decode_stages, in->decode_waves))
    return PF_ERR_INVALID;
  Tuning& t = tuning();
  t.tail_dynamic_pct = in->tail_dynamic_pct;
  t.decode_stages = in->decode_stages;
  t.decode_waves = in->decode_waves;
  return PF_OK;
}

int pf_attn_fwd(const pf_attn_fwd_args* a, void* stream) {
  if (!a) return PF_ERR_INVALID;
  pf::FwdParams p;
  int st = fill_fwd(a, &p);
  if (st != PF_OK) return st;
  if (p.n_work == 0) return PF_OK;
  p.tail = plan_tail(p.n_work, kTwoPerCu, (hipStream_t)stream);
  return finish(pf::launch_attn_fwd(p, a->dtype, a->head_dim, a->causal != 0, false,
                                    (hipStream_t)stream));
}

static size_t rope_ws_bytes(const pf_attn_fwd_args& b) {
  const size_t es = b.dtype == PF_DTYPE_F32 ? 4 : 2;
  return (((size_t)b.batch * b.num_kv_heads * b.seq_len_k * b.head_dim * es) + 255) & ~(size_t)255;
}

size_t pf_attn_fwd_rope_workspace_size(const pf_attn_fwd_rope_args* a) {
  if (!a) return 0;
  pf::FwdParams p;
  if (fill_fwd(&a->base, &p) != PF_OK) return 0;
  return rope_ws_bytes(a->base);
}

int pf_attn_fwd_rope(const pf_attn_fwd_rope_args* a, void* stream) {
  if (!a) return PF_ERR_INVALID;
  pf::FwdParams p;
  int st = fill_fwd(&a->base, &p);
  if (st != PF_OK) return st;
  if (!a->q_cos || !a->q_sin || !a->k_cos || !a->k_sin) return PF_ERR_INVALID;
  if (a->base.head_dim % 2 != 0) return PF_ERR_INVALID;  // fused_rope.py:168-169
  if (p.n_work == 0) return PF_OK;
  const size_t need = rope_ws_bytes(a->base);
  if (!a->workspace || a->workspace_bytes < need || ((uintptr_t)a->workspace & 255) != 0)
    return PF_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  st = finish(pf::launch_rope_rotate_k(a->base.k, a->workspace, a->k_cos, a->k_sin, a->base.batch,
                                       a->base.num_kv_heads, a->base.seq_len_k, a->base.kv_len,
                                       a->base.dtype, a->base.head_dim, s));
  if (st != PF_OK) return st;
  p.k = a->workspace;  // rotated K
  p.q_cos = a->q_cos;
  p.q_sin = a->q_sin;
  p.lse = nullptr;  // the reference's fused kernel has no LSE output
  p.tail = plan_tail(p.n_work, kTwoPerCu, s);
  return finish(pf::launch_attn_fwd(p, a->base.dtype, a->base.head_dim, a->base.causal != 0, true, s));
}

// ---------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------
static int fill_bwd(const pf_attn_bwd_args* a, pf::BwdParams* p, bool need_grads) {
  if (!a) return PF_ERR_INVALID;
  int st = check_attn_dims(a->batch, a->num_heads, a->num_kv_heads, a->seq_len_q, a->seq_len_k,
                           a->head_dim, a->kv_len, a->sm_scale, a->dtype);
  if (st != PF_OK) return st;
  if (!a->o || !a->do_ || !a->delta) return PF_ERR_INVALID;
  if (need_grads && (!a->q || !a->k || !a->v || !a->lse || !a->dq || !a->dk || !a->dv))
    return PF_ERR_INVALID;
  p->q = a->q;
  p->k = a->k;
  p->v = a->v;
  p->o = a->o;
  p->dout = a->do_;
  p->lse = a->lse;
  p->delta = a->delta;
  p->dq = a->dq;
  p->dk = a->dk;
  p->dv = a->dv;
  p->B = a->batch;
  p->Hq = a->num_heads;
  p->Hkv = a->num_kv_heads;
  p->Sq = a->seq_len_q;
  p->Sk = a->seq_len_k;
  p->kv_len = a->kv_len;
  p->g = a->num_heads / a->num_kv_heads;
  p->sm_scale = a->sm_scale;
  p->scale_log2 = a->sm_scale * 1.4426950408889634f;
  p->tail = pf::WorkTail{nullptr, 0, 0};
  const int64_t rows = (int64_t)a->batch * a->num_heads * a->seq_len_q;
  if (rows > kMaxGrid) return PF_ERR_UNSUPPORTED;
  // Per-(batch, head) byte offsets and buffer sizes are 32-bit inside the
  // kernels (Q/dO rows of one query head, K/V rows of one kv head), as in
  // the forward.
  const int64_t max_rows = a->seq_len_q > a->seq_len_k ? a->seq_len_q : a->seq_len_k;
  if ((max_rows + 256) * a->head_dim * 4 > 0x7fffffff) return PF_ERR_UNSUPPORTED;
  return PF_OK;
}

int pf_attn_bwd_delta(const pf_attn_bwd_args* a, void* stream) {
  pf::BwdParams p;
  int st = fill_bwd(a, &p, false);
  if (st != PF_OK) return st;
  if ((int64_t)p.B * p.Hq * p.Sq == 0) return PF_OK;
  return finish(pf::launch_attn_bwd_delta(p, a->dtype, a->head_dim, (hipStream_t)stream));
}

int pf_attn_bwd_dq(const pf_attn_bwd_args* a, void* stream) {
  pf::BwdParams p;
  int st = fill_bwd(a, &p, true);
  if (st != PF_OK) return st;
  if ((int64_t)p.B * p.Hq * p.Sq == 0) return PF_OK;
  p.tail = plan_tail(pf::bwd_dq_items(p), kTwoPerCu, (hipStream_t)stream);
  return finish(pf::launch_attn_bwd_dq(p, a->dtype, a->head_dim, a->causal != 0, (hipStream_t)stream));
}

int pf_attn_bwd_dkv(const pf_attn_bwd_args* a, void* stream) {
  pf::BwdParams p;
  int st = fill_bwd(a, &p, true);
  if (st != PF_OK) return st;
  if ((int64_t)p.B * p.Hkv * p.Sk == 0) return PF_OK;
  return finish(pf::launch_attn_bwd_dkv(p, a->dtype, a->head_dim, a->causal != 0, (hipStream_t)stream));
}

int pf_attn_bwd(const pf_attn_bwd_args* a, void* stream) {
  pf::BwdParams p;
  int st = fill_bwd(a, &p, true);
  if (st != PF_OK) return st;
  hipStream_t s = (hipStream_t)stream;
  if ((int64_t)p.B * p.Hq * p.Sq > 0) {
    // the dQ kernel computes delta itself and stores it for dK/dV
    p.tail = plan_tail(pf::bwd_dq_items(p), kTwoPerCu, s);
    st = finish(pf::launch_attn_bwd_dq(p, a->dtype, a->head_dim, a->causal != 0, s));
    if (st != PF_OK) return st;
  }
  if ((int64_t)p.B * p.Hkv * p.Sk > 0) {
    p.tail = pf::WorkTail{nullptr, 0, 0};  // dK/dV runs without a tail (plan_tail)
    st = finish(pf::launch_attn_bwd_dkv(p, a->dtype, a->head_dim, a->causal != 0, s));
  }
  return st;
}

// ---------------------------------------------------------------------------
// Decode (contiguous cache) and paged decode
// ---------------------------------------------------------------------------
static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Key-chunk size for split-KV: enough (b, kv head, chunk) waves to fill the
// chip several times over (256 CUs x 8 resident waves), chunks a multiple of
// the 64-key block and at least 256 keys so each wave streams a useful run.
static int decode_chunk(int64_t units, int max_len) {
  const int64_t target_waves = 4096;
  int64_t n_split = (target_waves + units - 1) / (units > 0 ? units : 1);
  if (n_split < 1) n_split = 1;
  int64_t chunk = (max_len + n_split - 1) / n_split;
  chunk = ((chunk + 63) / 64) * 64;
  if (chunk < 256) chunk = 256;
  return (int)chunk;
}

// Streaming kernel (decode_stream.hip): a persistent grid of one-wave
// workgroups, as many as are resident at once (queried once per device),
// with an LDS ring of 2 stages (measured on MI355X: 2 stages x 4 waves per
// CU beat 3 x 3 and 4 x 2). Tuning and test overrides: decode_stages (2..4)
// and decode_waves (grid size; any value >= 1 is correct, only the resident
// count is fast).
static int stream_setup(pf::DecodeParams* p, int group) {
  Tuning& t = tuning();
  const int ns = t.decode_stages.load(std::memory_order_relaxed);
  p->stages = ns;
  const int wv = t.decode_waves.load(std::memory_order_relaxed);
  p->n_waves = wv > 0 ? wv : pf::decode_stream_waves(ns, group);
  p->n_split = 0;
  p->chunk = 0;
  return p->n_waves;
}

static int fill_decode(const pf_attn_decode_args* a, pf::DecodeParams* p) {
  if (!a) return PF_ERR_INVALID;
  if (a->batch < 0 || a->num_heads < 1 || a->num_kv_heads < 1 || a->cache_size < 1)
    return PF_ERR_INVALID;
  if (a->num_heads % a->num_kv_heads != 0) return PF_ERR_INVALID;
  if (a->cache_len < 1 || a->cache_len > a->cache_size) return PF_ERR_INVALID;
  if (!isfinite(a->sm_scale)) return PF_ERR_INVALID;
  if (!dtype_ok(a->dtype)) return PF_ERR_UNSUPPORTED;
  if (!decode_head_dim_ok(a->head_dim, a->dtype)) return PF_ERR_UNSUPPORTED;
  const int g = a->num_heads / a->num_kv_heads;
  const int64_t units = (int64_t)a->batch * a->num_kv_heads * ((g + 31) / 32);
  *p = pf::DecodeParams{};
  p->q = a->q;
  p->k = a->k_cache;
  p->v = a->v_cache;
  p->o = a->o;
  p->B = a->batch;
  p->Hq = a->num_heads;
  p->Hkv = a->num_kv_heads;
  p->D = decode_compute_dim(a->head_dim);
  p->dr = a->head_dim;
  p->cache_size = a->cache_size;
  p->cache_len = a->cache_len;
  p->scale_log2 = a->sm_scale * 1.4426950408889634f;
  if (pf::decode_stream_supported(a->dtype, a->head_dim, false, 0)) {
    // buffer offsets within one (b, kv head) run are 32-bit
    if ((int64_t)a->cache_size * a->head_dim * 2 >= ((int64_t)1 << 31)) return PF_ERR_UNSUPPORTED;
    if (stream_setup(p, g) <= 0) return PF_ERR_LAUNCH;
    return PF_OK;
  }
  p->chunk = decode_chunk(units, a->cache_len);
  p->n_split = (a->cache_len + p->chunk - 1) / p->chunk;
  if (units * p->n_split > kMaxGrid) return PF_ERR_UNSUPPORTED;
  return PF_OK;
}

// Partial slots: streaming kernel 2 per wave x query rows; generic kernel
// one per (b, query head, chunk).
static size_t decode_slots(const pf::DecodeParams& p) {
  if (p.n_waves > 0) return (size_t)2 * p.n_waves * pf::decode_stream_qrows(p.Hq / p.Hkv);
  return (size_t)p.B * p.Hq * p.n_split;
}

static size_t decode_ws_bytes(const pf::DecodeParams& p) {
  const size_t slots = decode_slots(p);
  return align256(slots * p.D * sizeof(float)) + align256(slots * 2 * sizeof(float));
}

static int bind_workspace(pf::DecodeParams* p, void* ws, size_t bytes) {
  const size_t need = decode_ws_bytes(*p);
  if (need == 0) return PF_OK;
  if (!ws || bytes < need || ((uintptr_t)ws & 255) != 0) return PF_ERR_WORKSPACE;
  const size_t slots = decode_slots(*p);
  p->part_o = static_cast<float*>(ws);
  p->part_ml = reinterpret_cast<float*>(static_cast<char*>(ws) + align256(slots * p->D * sizeof(float)));
  return PF_OK;
}

size_t pf_attn_decode_workspace_size(const pf_attn_decode_args* a) {
  pf::DecodeParams p;
  if (fill_decode(a, &p) != PF_OK) return 0;
  return decode_ws_bytes(p);
}

int pf_attn_decode(const pf_attn_decode_args* a, void* stream) {
  pf::DecodeParams p;
  int st = fill_decode(a, &p);
  if (st != PF_OK) return st;
  if (!a->q || !a->k_cache || !a->v_cache || !a->o) return PF_ERR_INVALID;
  if (a->batch == 0) return PF_OK;
  st = bind_workspace(&p, a->workspace, a->workspace_bytes);
  if (st != PF_OK) return st;
  return finish(pf::launch_decode(p, a->dtype, false, (hipStream_t)stream));
}

static int fill_paged(const pf_paged_attn_args* a, pf::DecodeParams* p) {
  if (!a) return PF_ERR_INVALID;
  // paged.py:129-149: Sq == 1 (implied by the struct), heads divisible, table [B, P], lens [B].
  if (a->batch < 0 || a->num_heads < 1 || a->num_kv_heads < 1 || a->num_pages < 1 ||
      a->page_size < 1 || a->pages_per_seq < 0)
    return PF_ERR_INVALID;
  if (a->num_heads % a->num_kv_heads != 0) return PF_ERR_INVALID;
  if (!isfinite(a->sm_scale)) return PF_ERR_INVALID;
  if (!dtype_ok(a->dtype)) return PF_ERR_UNSUPPORTED;
  if (!decode_head_dim_ok(a->head_dim, a->dtype)) return PF_ERR_UNSUPPORTED;
  const int64_t max_len = (int64_t)a->pages_per_seq * a->page_size;
  if (max_len > 0x7fffffff) return PF_ERR_UNSUPPORTED;
  const int g = a->num_heads / a->num_kv_heads;
  const int64_t units = (int64_t)a->batch * a->num_kv_heads * ((g + 31) / 32);
  *p = pf::DecodeParams{};
  p->q = a->q;
  p->k = a->k_pages;
  p->v = a->v_pages;
  p->o = a->o;
  p->block_tables = a->block_tables;
  p->context_lens = a->context_lens;
  p->B = a->batch;
  p->Hq = a->num_heads;
  p->Hkv = a->num_kv_heads;
  p->D = decode_compute_dim(a->head_dim);
  p->dr = a->head_dim;
  p->num_pages = a->num_pages;
  p->page_size = a->page_size;
  p->pages_per_seq = a->pages_per_seq;
  p->scale_log2 = a->sm_scale * 1.4426950408889634f;
  if (pf::decode_stream_supported(a->dtype, a->head_dim, true, a->page_size)) {
    if ((int64_t)a->page_size * a->head_dim * 2 >= ((int64_t)1 << 31)) return PF_ERR_UNSUPPORTED;
    if (stream_setup(p, g) <= 0) return PF_ERR_LAUNCH;
    return PF_OK;
  }
  p->chunk = decode_chunk(units, (int)(max_len > 0 ? max_len : 1));
  p->n_split = max_len > 0 ? (int)((max_len + p->chunk - 1) / p->chunk) : 1;
  if (units * p->n_split > kMaxGrid) return PF_ERR_UNSUPPORTED;
  return PF_OK;
}

size_t pf_paged_attn_workspace_size(const pf_paged_attn_args* a) {
  pf::DecodeParams p;
  if (fill_paged(a, &p) != PF_OK) return 0;
  return decode_ws_bytes(p);
}

int pf_paged_attn(const pf_paged_attn_args* a, void* stream) {
  pf::DecodeParams p;
  int st = fill_paged(a, &p);
  if (st != PF_OK) return st;
  if (!a->q || !a->k_pages || !a->v_pages || !a->o || !a->context_lens) return PF_ERR_INVALID;
  if (a->pages_per_seq > 0 && !a->block_tables) return PF_ERR_INVALID;
  if (a->batch == 0) return PF_OK;
  st = bind_workspace(&p, a->workspace, a->workspace_bytes);
  if (st != PF_OK) return st;
  return finish(pf::launch_decode(p, a->dtype, true, (hipStream_t)stream));
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Paged decode with no caller workspace (pf_paged_attn_noalloc): the split-KV
// partials live in `scratch`, a file-scope device array that every GPU holds
// once, for the life of the process. On the host `scratch` names a host-side
// stand-in, not device memory: its device address is looked up once per
// device (hipGetSymbolAddress, with that device current) and only that
// address is handed to the kernels. Every call on one GPU shares the array;
// nothing in it needs clearing between calls (each launch writes every
// partial slot its combine step reads), and calls that overlap on one GPU
// (concurrent streams) race on it.
// ---------------------------------------------------------------------------
namespace {

static_assert(PF_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch keeps the workspace alignment");
static __device__ __align__(256) char scratch[PF_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;

struct ScratchAddr {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipErrorNotInitialized;
};
ScratchAddr g_scratch[kMaxScratchDevices];

// Device address of `scratch` on the device that `stream` belongs to (the
// null stream's: the current device), resolved on the first call on each
// device (symbol_address, with that device current, also under graph
// capture).
int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return PF_ERR_LAUNCH;
  ScratchAddr& s = g_scratch[dev];
  std::call_once(s.once, [&s, dev] { s.err = pf::symbol_address(dev, HIP_SYMBOL(scratch), &s.ptr); });
  if (s.err != hipSuccess || s.ptr == nullptr) return PF_ERR_LAUNCH;
  *out = s.ptr;
  return PF_OK;
}

}  // namespace

extern "C" {

int pf_paged_attn_noalloc(const pf_paged_attn_args* a, void* stream) {
  pf::DecodeParams p;
  int st = fill_paged(a, &p);
  if (st != PF_OK) return st;
  if (!a->q || !a->k_pages || !a->v_pages || !a->o || !a->context_lens) return PF_ERR_INVALID;
  if (a->pages_per_seq > 0 && !a->block_tables) return PF_ERR_INVALID;
  if (a->batch == 0) return PF_OK;
  const size_t need = decode_ws_bytes(p);
  if (need > (size_t)PF_NOALLOC_SCRATCH_BYTES) return PF_ERR_WORKSPACE;
  void* ws = nullptr;
  st = scratch_address((hipStream_t)stream, &ws);
  if (st != PF_OK) return st;
  st = bind_workspace(&p, ws, PF_NOALLOC_SCRATCH_BYTES);
  if (st != PF_OK) return st;
  return finish(pf::launch_decode(p, a->dtype, true, (hipStream_t)stream));
}

int pf_rope(const pf_rope_args* a, void* stream) {
  if (!a) return PF_ERR_INVALID;
  if (a->batch < 0 || a->heads < 0 || a->seq_len < 0 || a->head_dim < 2 || a->head_dim % 2 != 0)
    return PF_ERR_INVALID;
  if (a->inverse != 0 && a->inverse != 1) return PF_ERR_INVALID;
  if (!dtype_ok(a->dtype)) return PF_ERR_UNSUPPORTED;
  if (!head_dim_ok(a->head_dim, a->dtype)) return PF_ERR_UNSUPPORTED;
  if ((int64_t)a->batch * a->heads * a->seq_len == 0) return PF_OK;
  if (!a->x || !a->out || !a->cos || !a->sin || a->rope_len < a->seq_len) return PF_ERR_INVALID;
  return finish(pf::launch_rope_rotate_k(a->x, a->out, a->cos, a->sin, a->batch, a->heads, a->seq_len,
                                         a->seq_len, a->dtype, a->head_dim, (hipStream_t)stream,
                                         a->inverse != 0));
}

// ---------------------------------------------------------------------------
// Cache writes and the fused decode step
// ---------------------------------------------------------------------------
int pf_kv_cache_write(const pf_kv_cache_write_args* a, void* stream) {
  if (!a) return PF_ERR_INVALID;
  if (a->batch < 0 || a->num_kv_heads < 1 || a->seq_len < 0 || a->cache_size < 1) return PF_ERR_INVALID;
  if (a->positions_stride != 0 && a->positions_stride != 1) return PF_ERR_INVALID;
  if (a->ring != 0 && a->ring != 1) return PF_ERR_INVALID;
  if (!dtype_ok(a->dtype)) return PF_ERR_UNSUPPORTED;
  if (!decode_head_dim_ok(a->head_dim, a->dtype)) return PF_ERR_UNSUPPORTED;
  if ((int64_t)a->batch * a->num_kv_heads * a->seq_len == 0) return PF_OK;
  if (!a->k || !a->v || !a->k_cache || !a->v_cache || !a->positions) return PF_ERR_INVALID;
  pf::KvWriteParams p{a->k, a->v, a->k_cache, a->v_cache, a->positions, a->positions_stride,
                      a->batch, a->num_kv_heads, a->seq_len, a->cache_size, a->ring, a->head_dim};
  return finish(pf::launch_kv_cache_write(p, a->dtype, a->head_dim, (hipStream_t)stream));
}

int pf_paged_cache_write(const pf_paged_cache_write_args* a, void* stream) {
  if (!a) return PF_ERR_INVALID;
  if (a->batch < 0 || a->num_kv_heads < 1 || a->seq_len < 0 || a->num_pages < 1 || a->page_size < 1 ||
      a->pages_per_seq < 0)
    return PF_ERR_INVALID;
  if (a->positions_stride != 0 && a->positions_stride != 1) return PF_ERR_INVALID;
  if (!dtype_ok(a->dtype)) return PF_ERR_UNSUPPORTED;
  if (!decode_head_dim_ok(a->head_dim, a->dtype)) return PF_ERR_UNSUPPORTED;
  if ((int64_t)a->batch * a->num_kv_heads * a->seq_len == 0 || a->pages_per_seq == 0) return PF_OK;
  if (!a->k || !a->v || !a->k_pages || !a->v_pages || !a->positions || !a->block_tables) return PF_ERR_INVALID;
  pf::PagedWriteParams p{a->k, a->v, a->k_pages, a->v_pages, a->block_tables, a->positions,
                         a->positions_stride, a->batch, a->num_kv_heads, a->seq_len, a->num_pages,
                         a->page_size, a->pages_per_seq, a->head_dim};
  return finish(pf::launch_paged_cache_write(p, a->dtype, a->head_dim, (hipStream_t)stream));
}

// The fused decode step is one streaming-decode launch in its step mode
// (decode_stream.hip, PG == 1) plus the combine; its workspace is the split
// partials only.
static int fill_decode_step(const pf_attn_decode_step_args* a, pf::DecodeParams* p) {
  if (!a) return PF_ERR_INVALID;
  if (a->batch < 0 || a->num_heads < 1 || a->num_kv_heads < 1 || a->cache_size < 1) return PF_ERR_INVALID;
  if (a->num_heads % a->num_kv_heads != 0) return PF_ERR_INVALID;
  if (a->positions_stride != 0 && a->positions_stride != 1) return PF_ERR_INVALID;
  if (a->ring != 0 && a->ring != 1) return PF_ERR_INVALID;
  if ((a->cos == nullptr) != (a->sin == nullptr)) return PF_ERR_INVALID;
  if (a->cos != nullptr && a->rope_len < 1) return PF_ERR_INVALID;
  if (!isfinite(a->sm_scale)) return PF_ERR_INVALID;
  if (!dtype_ok(a->dtype)) return PF_ERR_UNSUPPORTED;
  if (!pf::decode_stream_supported(a->dtype, a->head_dim, false, 0)) return PF_ERR_UNSUPPORTED;
  if ((int64_t)a->cache_size * a->head_dim * 2 >= ((int64_t)1 << 31)) return PF_ERR_UNSUPPORTED;
  *p = pf::DecodeParams{};
  p->q = a->q;
  p->k = a->k_cache;
  p->v = a->v_cache;
  p->o = a->o;
  p->B = a->batch;
  p->Hq = a->num_heads;
  p->Hkv = a->num_kv_heads;
  p->D = decode_compute_dim(a->head_dim);
  p->dr = a->head_dim;
  p->cache_size = a->cache_size;
  p->cache_len = a->cache_size;
  p->scale_log2 = a->sm_scale * 1.4426950408889634f;
  p->positions = a->positions;
  p->pos_stride = a->positions_stride;
  p->ring = a->ring;
  p->rope_cos = a->cos;
  p->rope_sin = a->sin;
  p->rope_len = a->rope_len;
  p->k_new = a->k_new;
  p->v_new = a->v_new;
  p->k_out = a->k_cache;
  p->v_out = a->v_cache;
  if (stream_setup(p, a->num_heads / a->num_kv_heads) <= 0) return PF_ERR_LAUNCH;
  return PF_OK;
}

size_t pf_attn_decode_step_workspace_size(const pf_attn_decode_step_args* a) {
  pf::DecodeParams p;
  if (fill_decode_step(a, &p) != PF_OK) return 0;
  return decode_ws_bytes(p);
}

int pf_attn_decode_step(const pf_attn_decode_step_args* a, void* stream) {
  pf::DecodeParams p;
  int st = fill_decode_step(a, &p);
  if (st != PF_OK) return st;
  if (a->batch == 0) return PF_OK;
  if (!a->q || !a->k_new || !a->v_new || !a->k_cache || !a->v_cache || !a->o || !a->positions)
    return PF_ERR_INVALID;
  st = bind_workspace(&p, a->workspace, a->workspace_bytes);
  if (st != PF_OK) return st;
  return finish(pf::launch_decode(p, a->dtype, false, (hipStream_t)stream));
}

}  // extern "C"
