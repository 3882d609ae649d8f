// Host-side validation of the C ABI under AddressSanitizer and
// UndefinedBehaviorSanitizer (built by `make asan` in the package directory;
// run on a machine with or without a GPU: no call below reaches a launch).
//
// Every entry point is called with a NULL argument block and with argument
// blocks that the host validation must refuse (shapes, scalars, dtypes, head
// dims, workspace sizes, 32-bit range limits), the pure-host queries run on
// valid shapes, and the tuning round trip is exercised. The program prints
// one line per failed expectation and exits non-zero if any failed; the
// sanitizers abort on any memory or UB error in the host code.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "pallas_flash_amd.h"

static int g_fail = 0;

#define EXPECT(cond, what)                                  \
  do {                                                      \
    if (!(cond)) {                                          \
      printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, what); \
      ++g_fail;                                             \
    }                                                       \
  } while (0)

// Distinct non-null "device" addresses: validation only compares them with
// NULL and checks their alignment, so they are never dereferenced.
static void* fake(uintptr_t i) { return (void*)(uintptr_t)(0x100000 + 256 * i); }

static pf_attn_fwd_args fwd_ok() {
  pf_attn_fwd_args a;
  memset(&a, 0, sizeof a);
  a.q = fake(1); a.k = fake(2); a.v = fake(3); a.o = fake(4); a.lse = NULL;
  a.batch = 1; a.num_heads = 4; a.num_kv_heads = 2; a.seq_len_q = 16; a.seq_len_k = 16;
  a.head_dim = 128; a.kv_len = 16; a.causal = 0; a.sm_scale = 0.1f; a.dtype = PF_DTYPE_BF16;
  return a;
}

static void test_fwd() {
  EXPECT(pf_attn_fwd(NULL, NULL) == PF_ERR_INVALID, "fwd NULL args");
  struct { void (*edit)(pf_attn_fwd_args*); int want; const char* name; } cases[] = {
      {[](pf_attn_fwd_args* a) { a->num_heads = 6; a->num_kv_heads = 4; }, PF_ERR_INVALID, "fwd heads"},
      {[](pf_attn_fwd_args* a) { a->num_kv_heads = 0; }, PF_ERR_INVALID, "fwd zero kv heads"},
      {[](pf_attn_fwd_args* a) { a->kv_len = 0; }, PF_ERR_INVALID, "fwd kv_len 0"},
      {[](pf_attn_fwd_args* a) { a->kv_len = 17; }, PF_ERR_INVALID, "fwd kv_len > Sk"},
      {[](pf_attn_fwd_args* a) { a->batch = -1; }, PF_ERR_INVALID, "fwd negative batch"},
      {[](pf_attn_fwd_args* a) { a->sm_scale = NAN; }, PF_ERR_INVALID, "fwd NaN scale"},
      {[](pf_attn_fwd_args* a) { a->sm_scale = INFINITY; }, PF_ERR_INVALID, "fwd inf scale"},
      {[](pf_attn_fwd_args* a) { a->q = NULL; }, PF_ERR_INVALID, "fwd NULL q"},
      {[](pf_attn_fwd_args* a) { a->o = NULL; }, PF_ERR_INVALID, "fwd NULL o"},
      {[](pf_attn_fwd_args* a) { a->dtype = 7; }, PF_ERR_UNSUPPORTED, "fwd dtype"},
      {[](pf_attn_fwd_args* a) { a->head_dim = 96; }, PF_ERR_UNSUPPORTED, "fwd head_dim"},
      {[](pf_attn_fwd_args* a) { a->seq_len_k = a->kv_len = 1 << 24; }, PF_ERR_UNSUPPORTED, "fwd 32-bit range"},
      {[](pf_attn_fwd_args* a) { a->batch = 1 << 20; a->seq_len_q = 1 << 20; }, PF_ERR_UNSUPPORTED, "fwd grid size"},
  };
  for (auto& c : cases) {
    pf_attn_fwd_args a = fwd_ok();
    c.edit(&a);
    EXPECT(pf_attn_fwd(&a, NULL) == c.want, c.name);
  }
}

static void test_rope() {
  EXPECT(pf_attn_fwd_rope(NULL, NULL) == PF_ERR_INVALID, "rope NULL args");
  EXPECT(pf_attn_fwd_rope_workspace_size(NULL) == 0, "rope ws NULL");
  pf_attn_fwd_rope_args r;
  memset(&r, 0, sizeof r);
  r.base = fwd_ok();
  r.q_cos = r.q_sin = r.k_cos = r.k_sin = (const float*)fake(9);
  const size_t ws = pf_attn_fwd_rope_workspace_size(&r);
  EXPECT(ws >= (size_t)1 * 2 * 16 * 128 * 2, "rope workspace covers rotated K");
  r.workspace = NULL;
  r.workspace_bytes = ws;
  EXPECT(pf_attn_fwd_rope(&r, NULL) == PF_ERR_WORKSPACE, "rope NULL workspace");
  r.workspace = fake(10);
  r.workspace_bytes = ws - 1;
  EXPECT(pf_attn_fwd_rope(&r, NULL) == PF_ERR_WORKSPACE, "rope small workspace");
  r.workspace = (void*)((uintptr_t)fake(10) + 4);
  r.workspace_bytes = ws;
  EXPECT(pf_attn_fwd_rope(&r, NULL) == PF_ERR_WORKSPACE, "rope misaligned workspace");
  r.q_cos = NULL;
  EXPECT(pf_attn_fwd_rope(&r, NULL) == PF_ERR_INVALID, "rope NULL table");

  pf_rope_args x;
  memset(&x, 0, sizeof x);
  EXPECT(pf_rope(NULL, NULL) == PF_ERR_INVALID, "pf_rope NULL args");
  x.x = fake(1); x.out = fake(2); x.cos = x.sin = (const float*)fake(3);
  x.batch = 1; x.heads = 2; x.seq_len = 8; x.head_dim = 128; x.rope_len = 4; x.dtype = PF_DTYPE_BF16;
  EXPECT(pf_rope(&x, NULL) == PF_ERR_INVALID, "pf_rope table shorter than seq_len");
}

static pf_attn_bwd_args bwd_ok() {
  pf_attn_bwd_args a;
  memset(&a, 0, sizeof a);
  a.q = fake(1); a.k = fake(2); a.v = fake(3); a.o = fake(4); a.do_ = fake(5);
  a.lse = (const float*)fake(6); a.delta = (float*)fake(7);
  a.dq = fake(8); a.dk = fake(9); a.dv = fake(10);
  a.batch = 1; a.num_heads = 4; a.num_kv_heads = 2; a.seq_len_q = 16; a.seq_len_k = 16;
  a.head_dim = 128; a.kv_len = 16; a.causal = 1; a.sm_scale = 0.1f; a.dtype = PF_DTYPE_BF16;
  return a;
}

static void test_bwd() {
  int (*fns[])(const pf_attn_bwd_args*, void*) = {pf_attn_bwd, pf_attn_bwd_delta, pf_attn_bwd_dq, pf_attn_bwd_dkv};
  for (auto f : fns) {
    EXPECT(f(NULL, NULL) == PF_ERR_INVALID, "bwd NULL args");
    pf_attn_bwd_args a = bwd_ok();
    a.kv_len = 0;
    EXPECT(f(&a, NULL) == PF_ERR_INVALID, "bwd kv_len");
    a = bwd_ok();
    a.delta = NULL;
    EXPECT(f(&a, NULL) == PF_ERR_INVALID, "bwd NULL delta");
    a = bwd_ok();
    a.head_dim = 80;
    EXPECT(f(&a, NULL) == PF_ERR_UNSUPPORTED, "bwd head_dim");
    a = bwd_ok();
    a.seq_len_q = 1 << 22;
    EXPECT(f(&a, NULL) == PF_ERR_UNSUPPORTED, "bwd 32-bit range");
  }
}

static pf_attn_decode_args dec_ok() {
  pf_attn_decode_args a;
  memset(&a, 0, sizeof a);
  a.q = fake(1); a.k_cache = fake(2); a.v_cache = fake(3); a.o = fake(4);
  a.batch = 2; a.num_heads = 8; a.num_kv_heads = 2; a.cache_size = 64; a.head_dim = 128;
  a.cache_len = 40; a.sm_scale = 0.1f; a.dtype = PF_DTYPE_BF16;
  return a;
}

static void test_decode() {
  EXPECT(pf_attn_decode(NULL, NULL) == PF_ERR_INVALID, "decode NULL args");
  EXPECT(pf_attn_decode_workspace_size(NULL) == 0, "decode ws NULL");
  pf_attn_decode_args a = dec_ok();
  const size_t ws = pf_attn_decode_workspace_size(&a);
  EXPECT(ws > 0, "decode workspace size");
  a.workspace = fake(5);
  a.workspace_bytes = ws - 1;
  EXPECT(pf_attn_decode(&a, NULL) == PF_ERR_WORKSPACE, "decode small workspace");
  a = dec_ok();
  a.cache_len = 65;
  EXPECT(pf_attn_decode(&a, NULL) == PF_ERR_INVALID, "decode cache_len");
  EXPECT(pf_attn_decode_workspace_size(&a) == 0, "decode ws of invalid args");
  a = dec_ok();
  a.head_dim = 96;
  EXPECT(pf_attn_decode_workspace_size(&a) > 0, "decode head_dim 96 in place");
  a.head_dim = 100;
  EXPECT(pf_attn_decode(&a, NULL) == PF_ERR_UNSUPPORTED, "decode head_dim 100 (bf16)");
  a.dtype = PF_DTYPE_F32;
  EXPECT(pf_attn_decode_workspace_size(&a) > 0, "decode head_dim 100 (float32) in place");
}

static pf_paged_attn_args paged_ok() {
  pf_paged_attn_args a;
  memset(&a, 0, sizeof a);
  a.q = fake(1); a.k_pages = fake(2); a.v_pages = fake(3);
  a.block_tables = (const int32_t*)fake(4); a.context_lens = (const int32_t*)fake(5); a.o = fake(6);
  a.batch = 3; a.num_heads = 8; a.num_kv_heads = 2; a.num_pages = 32; a.page_size = 16; a.head_dim = 128;
  a.pages_per_seq = 4; a.sm_scale = 0.1f; a.dtype = PF_DTYPE_BF16;
  return a;
}

static void test_paged() {
  EXPECT(pf_paged_attn(NULL, NULL) == PF_ERR_INVALID, "paged NULL args");
  EXPECT(pf_paged_attn_noalloc(NULL, NULL) == PF_ERR_INVALID, "paged noalloc NULL args");
  EXPECT(pf_paged_attn_workspace_size(NULL) == 0, "paged ws NULL");
  pf_paged_attn_args a = paged_ok();
  const size_t ws = pf_paged_attn_workspace_size(&a);
  EXPECT(ws > 0, "paged workspace size");
  a.workspace = fake(7);
  a.workspace_bytes = ws - 1;
  EXPECT(pf_paged_attn(&a, NULL) == PF_ERR_WORKSPACE, "paged small workspace");
  a = paged_ok();
  a.page_size = 0;
  EXPECT(pf_paged_attn(&a, NULL) == PF_ERR_INVALID, "paged page_size 0");
  a = paged_ok();
  a.num_heads = 6; a.num_kv_heads = 4;
  EXPECT(pf_paged_attn(&a, NULL) == PF_ERR_INVALID, "paged heads");
  EXPECT(pf_paged_attn_noalloc(&a, NULL) == PF_ERR_INVALID, "paged noalloc heads");
  a = paged_ok();
  a.block_tables = NULL;
  EXPECT(pf_paged_attn(&a, NULL) == PF_ERR_INVALID, "paged NULL table");
}

static void test_cache_writes() {
  EXPECT(pf_kv_cache_write(NULL, NULL) == PF_ERR_INVALID, "kv write NULL args");
  pf_kv_cache_write_args w;
  memset(&w, 0, sizeof w);
  w.k = fake(1); w.v = fake(2); w.k_cache = fake(3); w.v_cache = fake(4); w.positions = (const int32_t*)fake(5);
  w.batch = 1; w.num_kv_heads = 2; w.seq_len = 4; w.cache_size = 16; w.head_dim = 128; w.dtype = PF_DTYPE_BF16;
  w.positions_stride = -1;
  EXPECT(pf_kv_cache_write(&w, NULL) == PF_ERR_INVALID, "kv write negative stride");
  w.positions_stride = 0;
  w.head_dim = 44;  // rows of whole 16-byte chunks only
  EXPECT(pf_kv_cache_write(&w, NULL) == PF_ERR_UNSUPPORTED, "kv write head_dim");
  w.head_dim = 264;
  EXPECT(pf_kv_cache_write(&w, NULL) == PF_ERR_UNSUPPORTED, "kv write head_dim above 256");

  EXPECT(pf_paged_cache_write(NULL, NULL) == PF_ERR_INVALID, "paged write NULL args");
  pf_paged_cache_write_args p;
  memset(&p, 0, sizeof p);
  p.k = fake(1); p.v = fake(2); p.k_pages = fake(3); p.v_pages = fake(4);
  p.block_tables = (const int32_t*)fake(5); p.positions = (const int32_t*)fake(6);
  p.batch = 1; p.num_kv_heads = 2; p.seq_len = 4; p.num_pages = 8; p.page_size = 0; p.head_dim = 128;
  p.pages_per_seq = 2; p.dtype = PF_DTYPE_BF16;
  EXPECT(pf_paged_cache_write(&p, NULL) == PF_ERR_INVALID, "paged write page_size 0");
}

static void test_decode_step() {
  EXPECT(pf_attn_decode_step(NULL, NULL) == PF_ERR_INVALID, "step NULL args");
  EXPECT(pf_attn_decode_step_workspace_size(NULL) == 0, "step ws NULL");
  pf_attn_decode_step_args s;
  memset(&s, 0, sizeof s);
  s.q = fake(1); s.k_new = fake(2); s.v_new = fake(3); s.k_cache = fake(4); s.v_cache = fake(5); s.o = fake(6);
  s.positions = (const int32_t*)fake(7); s.positions_stride = 1;
  s.cos = (const float*)fake(8); s.sin = NULL; s.rope_len = 64;
  s.batch = 2; s.num_heads = 8; s.num_kv_heads = 2; s.cache_size = 64; s.head_dim = 128;
  s.sm_scale = 0.1f; s.dtype = PF_DTYPE_BF16;
  EXPECT(pf_attn_decode_step(&s, NULL) == PF_ERR_INVALID, "step one table NULL");
  s.sin = (const float*)fake(9);
  const size_t ws = pf_attn_decode_step_workspace_size(&s);
  EXPECT(ws > 0, "step workspace size");
  s.dtype = PF_DTYPE_F32;
  EXPECT(pf_attn_decode_step(&s, NULL) == PF_ERR_UNSUPPORTED, "step float32");
}

static void test_tuning_and_version() {
  pf_tuning t, u;
  EXPECT(pf_get_tuning(NULL) == PF_ERR_INVALID, "get_tuning NULL");
  EXPECT(pf_set_tuning(NULL) == PF_ERR_INVALID, "set_tuning NULL");
  EXPECT(pf_get_tuning(&t) == PF_OK, "get_tuning");
  u = t;
  u.tail_dynamic_pct = 101;
  EXPECT(pf_set_tuning(&u) == PF_ERR_INVALID, "set_tuning dynamic share");
  u = t;
  u.decode_stages = 5;
  EXPECT(pf_set_tuning(&u) == PF_ERR_INVALID, "set_tuning stages");
  u = t;
  u.decode_waves = 7;
  EXPECT(pf_set_tuning(&u) == PF_OK, "set_tuning waves");
  pf_tuning v;
  EXPECT(pf_get_tuning(&v) == PF_OK && v.decode_waves == 7, "tuning round trip");
  EXPECT(pf_set_tuning(&t) == PF_OK, "tuning restore");
  const char* ver = pf_version();
  EXPECT(ver != NULL && strstr(ver, "gfx950") != NULL, "version string");
}

int main() {
  test_fwd();
  test_rope();
  test_bwd();
  test_decode();
  test_paged();
  test_cache_writes();
  test_decode_step();
  test_tuning_and_version();
  printf("%s: %d failed expectations\n", g_fail ? "FAIL" : "OK", g_fail);
  return g_fail ? 1 : 0;
}
