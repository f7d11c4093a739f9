// Entry points whose kernels are not built yet: they report DSA_ERR_UNSUPPORTED.
#include "dsa_common.h"

extern "C" int dsa_compressor_fwd(const float*, const float*, const float*, const float*, void*, int, int64_t,
                                  int64_t, int64_t, int64_t, int, float, void*) {
  return dsa::set_error(DSA_ERR_UNSUPPORTED, "dsa_compressor_fwd: not built yet");
}
