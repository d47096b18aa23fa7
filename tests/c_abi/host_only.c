/* A C99 client of include/llk/llk_abi.h: host-only calls (no GPU) that a
 * C caller -- or another language's FFI -- would make.  Exits non-zero on
 * the first failed check. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "llk/llk_abi.h"

#define CHECK(c)                                                          \
  do {                                                                    \
    if (!(c)) {                                                           \
      fprintf(stderr, "check failed at line %d: %s (%s)\n", __LINE__, #c, \
              llk_last_error());                                          \
      return 1;                                                           \
    }                                                                     \
  } while (0)

static int fake_entry(const llk_tensor2d* x, const llk_packed_weights* w0,
                      const llk_packed_weights* w1, llk_tensor2d* y, int y_dtype,
                      llk_kernel_context* ctx) {
  (void)x; (void)w0; (void)w1; (void)y; (void)y_dtype; (void)ctx;
  return LLK_OK;
}

/* The KernelFn-shaped entry point has exactly the reference's type
 * (JitCache.h:79-81) and MemRef2D is 56 bytes (JitCache.h:43-51). */
static const llk_memref_kernel_fn kernel_fn_shape = &llk_swiglu_kernel_fn;
typedef char memref_is_56_bytes[sizeof(llk_memref2d) == 56 ? 1 : -1];

int main(void) {
  const int64_t K = 100, N = 150, BK = 64;
  uint16_t* w = malloc((size_t)(K * N) * sizeof(uint16_t));
  int64_t i;
  memref_is_56_bytes* unused_size_check = NULL;
  llk_tensor2d wt;
  llk_packed_weights* pw = NULL;
  llk_packed_weights* back = NULL;
  size_t len = 0;
  void* blob;
  llk_launch_plan plan;
  llk_jit_cache* cache = NULL;
  llk_kernel_key key;
  llk_kernel_fn fn = NULL;
  llk_memref_kernel_fn kfn = NULL;
  llk_weight_key wk;
  (void)unused_size_check;
  CHECK(kernel_fn_shape != NULL);
  llk_packed_weights* hit = NULL;
  llk_cache_stats st;
  llk_schedule_entry se;
  int n = 0;

  CHECK(w != NULL);
  for (i = 0; i < K * N; ++i) w[i] = (uint16_t)(0x3f80 + (i % 97));
  CHECK(llk_abi_version() == LLK_ABI_VERSION);

  /* packWeightMatrix metadata (PackedWeights.cpp:5-15) */
  wt.data = w; wt.dim0 = K; wt.dim1 = N; wt.stride0 = N; wt.stride1 = 1;
  CHECK(llk_pack_weights(&wt, BK, LLK_PACK_HOST_ONLY, &pw) == LLK_OK);
  CHECK(llk_packed_weights_k_blocks(pw) == 2 && llk_packed_weights_n(pw) == N);
  CHECK(llk_packed_weights_block_size(pw) == BK * N * 2 && llk_packed_weights_bk(pw) == BK);
  CHECK(llk_packed_weights_dtype(pw) == LLK_BF16 && llk_packed_weights_host_data(pw) != NULL);

  /* blob round trip */
  CHECK(llk_packed_weights_serialize(pw, NULL, 0, &len) == LLK_OK);
  CHECK(len == 96 + llk_pack_device_bytes(K, N));
  blob = malloc(len);
  CHECK(blob != NULL);
  CHECK(llk_packed_weights_serialize(pw, blob, len, &len) == LLK_OK);
  CHECK(llk_packed_weights_deserialize(blob, len, LLK_PACK_HOST_ONLY, &back) == LLK_OK);
  CHECK(memcmp(llk_packed_weights_host_data(back), llk_packed_weights_host_data(pw),
               (size_t)(2 * BK * N) * sizeof(uint16_t)) == 0);
  ((unsigned char*)blob)[120] ^= 1u;
  CHECK(llk_packed_weights_deserialize(blob, len, LLK_PACK_HOST_ONLY, &hit) == LLK_ERR_INVALID_ARGUMENT);
  llk_packed_weights_free(back);
  free(blob);

  /* verifiers and planning */
  CHECK(llk_verify_fused_swiglu(2, 4, 4, 8, 4, 8, 3, 8) == LLK_ERR_SHAPE);
  CHECK(strstr(llk_last_error(), "M dimension mismatch") != NULL);
  CHECK(llk_classify_m(1) == 0 && llk_classify_m(4097) == 4);
  CHECK(llk_describe_launch(0, 2048, 11008, 4096, LLK_PLAN_X_ALIGNED, &plan) == LLK_OK);
  CHECK(plan.kernel == 2 && plan.workgroups == 504 && plan.workspace_bytes == 0 &&
        plan.tile_columns == 176);
  CHECK(llk_describe_launch(0, 2048, 11008, 4096, LLK_PLAN_X_ALIGNED | LLK_PLAN_OUT_F32, &plan) ==
        LLK_OK);
  CHECK(plan.kernel == 1 && plan.workgroups == 688 && plan.tile_columns == 128);
  /* the accumulating matmul always has its planes and the reduce launch */
  CHECK(llk_describe_launch(3, 700, 384, 768, LLK_PLAN_X_ALIGNED | LLK_PLAN_ACCUMULATE, &plan) ==
        LLK_OK);
  CHECK(plan.workspace_bytes > 0 && plan.launches == 2);
  CHECK(llk_describe_launch(0, 8, 8, 8, LLK_PLAN_ACCUMULATE, &plan) == LLK_ERR_INVALID_ARGUMENT);
  CHECK(llk_select_schedule("/nonexistent.json", "fused_swiglu", 0, &se, &n) == LLK_ERR_NOT_FOUND);
  CHECK(se.BM == 8 && se.BN == 32 && n == 0); /* built-in default */

  /* cache: L3 entry for a gfx950 key, L4 ownership */
  CHECK(llk_cache_create(&cache) == LLK_OK);
  memset(&key, 0, sizeof key);
  key.operation = 0; key.N = N; key.K = K; key.isa = 7; key.weight_layout = 2;
  key.thread_count = 1;
  /* the key's code object is missing from this directory: a status, and
     nothing is cached */
  CHECK(llk_cache_set_object_dir(cache, "/nonexistent-llk-objects") == LLK_OK);
  CHECK(llk_cache_lookup_or_compile(cache, &key, &kfn) == LLK_ERR_NOT_FOUND);
  CHECK(strstr(llk_last_error(), "/nonexistent-llk-objects/llk_fused_swiglu_gfx950.hsaco") != NULL);
  CHECK(llk_cache_lookup_object_code(cache, &key, &fn) == 0);
  /* the default directory (objects/ beside the library): read and checked
     on this host, loaded on a device at the entry's first call */
  CHECK(llk_cache_set_object_dir(cache, NULL) == LLK_OK);
  CHECK(llk_cache_lookup_or_compile(cache, &key, &kfn) == LLK_OK && kfn != NULL &&
        kfn != llk_swiglu_kernel_fn);
  CHECK(llk_cache_lookup_or_compile_packed(cache, &key, &fn) == LLK_OK && fn != NULL &&
        fn != llk_swiglu_bf16);
  CHECK(llk_cache_lookup_object_code(cache, &key, &fn) == 1);
  key.M_bucket = 3;
  CHECK(llk_cache_insert_object_code(cache, &key, fake_entry) == LLK_OK);
  CHECK(llk_cache_lookup_object_code(cache, &key, &fn) == 1 && fn == fake_entry);
  memset(&wk, 0, sizeof wk);
  wk.weight_ptr = w; wk.shape_hash = 1; wk.BK = BK; wk.BN = 128;
  CHECK(llk_cache_insert_packed_weights(cache, &wk, pw) == LLK_OK); /* cache owns pw */
  CHECK(llk_cache_lookup_packed_weights(cache, &wk, &hit) == 1 && hit == pw);
  CHECK(llk_cache_get_stats(cache, &st) == LLK_OK);
  CHECK(st.hits[2] == 3 && st.misses[2] == 3 && st.hits[3] == 1);
  CHECK(llk_cache_size(cache) == 3);
  llk_cache_destroy(cache); /* frees pw */
  free(w);
  printf("c abi ok\n");
  return 0;
}
