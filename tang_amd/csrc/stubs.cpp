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
}
