// Entry points whose implementation is not built yet: they fail loudly.
#include "capi_util.hpp"

#define TH_UNSUPPORTED(name) throw ::th::Error(TH_ERR_UNSUPPORTED, name ": not implemented")

extern "C" {
int th_mla_decode(th_device*, const th_buffer*, const th_buffer*, const th_buffer*, size_t, size_t, size_t, size_t, size_t,
                  size_t, size_t, const th_qweight*, const th_qweight*, float, th_buffer*) { TH_API_BEGIN TH_UNSUPPORTED("th_mla_decode"); TH_API_END }
}
