// Entry points whose implementation is not built yet: they fail loudly.
#include "capi_util.hpp"

#define TH_UNSUPPORTED(name) throw ::th::Error(TH_ERR_UNSUPPORTED, name ": not implemented")

extern "C" {
int th_moe_create(th_device*, size_t, size_t, size_t, size_t, size_t, th_moe**) { TH_API_BEGIN TH_UNSUPPORTED("th_moe_create"); TH_API_END }
int th_moe_destroy(th_moe*) { TH_API_BEGIN TH_UNSUPPORTED("th_moe_destroy"); TH_API_END }
int th_moe_init_synthetic(th_moe*, uint64_t) { TH_API_BEGIN TH_UNSUPPORTED("th_moe_init_synthetic"); TH_API_END }
int th_moe_forward(th_moe*, const th_buffer*, size_t, th_buffer*, th_buffer*, th_buffer*) { TH_API_BEGIN TH_UNSUPPORTED("th_moe_forward"); TH_API_END }
int th_mla_decode(th_device*, const th_buffer*, const th_buffer*, const th_buffer*, size_t, size_t, size_t, size_t, size_t,
                  size_t, size_t, const th_qweight*, const th_qweight*, float, th_buffer*) { TH_API_BEGIN TH_UNSUPPORTED("th_mla_decode"); TH_API_END }
int th_llama_create(th_device*, const th_llama_config*, th_llama**) { TH_API_BEGIN TH_UNSUPPORTED("th_llama_create"); TH_API_END }
int th_llama_destroy(th_llama*) { TH_API_BEGIN TH_UNSUPPORTED("th_llama_destroy"); TH_API_END }
int th_llama_init_synthetic(th_llama*, uint64_t) { TH_API_BEGIN TH_UNSUPPORTED("th_llama_init_synthetic"); TH_API_END }
int th_llama_fill_kv_synthetic(th_llama*, size_t, uint64_t) { TH_API_BEGIN TH_UNSUPPORTED("th_llama_fill_kv_synthetic"); TH_API_END }
int th_llama_generate(th_llama*, int32_t, size_t, size_t, int32_t*, float*) { TH_API_BEGIN TH_UNSUPPORTED("th_llama_generate"); TH_API_END }
int th_llama_step_device(th_llama*, size_t) { TH_API_BEGIN TH_UNSUPPORTED("th_llama_step_device"); TH_API_END }
int th_llama_set_token(th_llama*, int32_t) { TH_API_BEGIN TH_UNSUPPORTED("th_llama_set_token"); TH_API_END }
}
