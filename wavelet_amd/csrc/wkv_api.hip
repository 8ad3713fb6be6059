// Host-side plumbing of libwkv: error state, descriptor validation, version.
#include "wkv_common.h"

namespace wkv {

static thread_local char g_error[512] = "";

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_cache(const wkv_cache_t *c, int want_dtype) {
  WKV_CHECK_ARG(c != nullptr, "cache descriptor is NULL");
  WKV_CHECK_ARG(c->k != nullptr && c->v != nullptr, "cache k/v pointer is NULL");
  WKV_CHECK_ARG(aligned16(c->k) && aligned16(c->v), "cache k/v must be 16-byte aligned");
  WKV_CHECK_ARG(c->num_blocks > 0, "num_blocks must be positive (got %lld)", (long long)c->num_blocks);
  WKV_CHECK_ARG(c->block_size > 0 && c->block_size % 16 == 0 && c->block_size <= 256,
                "block_size must be a multiple of 16 in [16, 256] (got %d)", c->block_size);
  WKV_CHECK_ARG(c->num_kv_heads > 0, "num_kv_heads must be positive (got %d)", c->num_kv_heads);
  WKV_CHECK_ARG(c->kv_dtype == WKV_KV_BF16 || c->kv_dtype == WKV_KV_FP8_E4M3, "unknown kv_dtype %d",
                c->kv_dtype);
  WKV_CHECK_ARG((c->flags & ~WKV_CACHE_SHARED_BLOCKS) == 0, "unknown cache flags 0x%x",
                static_cast<unsigned>(c->flags & ~WKV_CACHE_SHARED_BLOCKS));
  WKV_CHECK_ARG(c->reserved == 0, "cache descriptor field `reserved` must be 0 (got %d)", c->reserved);
  if (c->head_dim != 64 && c->head_dim != 128)
    return fail(WKV_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", c->head_dim);
  if (want_dtype >= 0)
    WKV_CHECK_ARG(c->kv_dtype == want_dtype, "this entry point needs a %s cache (got %s)",
                  want_dtype == WKV_KV_BF16 ? "bf16" : "fp8_e4m3",
                  c->kv_dtype == WKV_KV_BF16 ? "bf16" : "fp8_e4m3");
  if (c->kv_dtype == WKV_KV_FP8_E4M3)
    WKV_CHECK_ARG(c->k_scale != nullptr && c->v_scale != nullptr, "fp8 cache needs k_scale and v_scale");
  return WKV_OK;
}

int check_mla_cache(const wkv_mla_cache_t *c) {
  WKV_CHECK_ARG(c != nullptr && c->latent != nullptr, "MLA cache is NULL");
  WKV_CHECK_ARG(aligned16(c->latent), "MLA latent cache must be 16-byte aligned");
  WKV_CHECK_ARG(c->num_blocks > 0 && c->block_size > 0 && c->block_size % 16 == 0 && c->block_size <= 256,
                "MLA cache needs num_blocks > 0 and block_size a multiple of 16 in [16, 256]");
  WKV_CHECK_ARG(c->kv_lora_rank % 8 == 0 && c->rope_dim % 8 == 0 && c->kv_lora_rank > 0 && c->rope_dim >= 0,
                "kv_lora_rank and rope_dim must be multiples of 8");
  return WKV_OK;
}

}  // namespace wkv

extern "C" const char *wkv_last_error(void) { return wkv::g_error; }

extern "C" int wkv_version(void) { return WKV_ABI_VERSION; }
