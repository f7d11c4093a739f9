// Entry points whose kernels are not built yet: they report DSA_ERR_UNSUPPORTED.
#include "dsa_common.h"

extern "C" int64_t dsa_sparse_mla_bwd_workspace_size(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t) { return 0; }
extern "C" int dsa_sparse_mla_bwd(const void*, const void*, const int32_t*, const void*, const void*, const float*,
                                  const float*, void*, float*, void*, int64_t, int, int64_t, int64_t, int64_t,
                                  int64_t, int64_t, int64_t, int64_t, float, int64_t, void*) {
  return dsa::set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_bwd: not built yet");
}
extern "C" int dsa_attn_mass(const void*, const void*, const int32_t*, const float*, const float*, float*, int,
                             int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, float, int64_t, void*) {
  return dsa::set_error(DSA_ERR_UNSUPPORTED, "dsa_attn_mass: not built yet");
}
extern "C" int dsa_indexer_kl_grad(const void*, const void*, const float*, const int32_t*, const float*, float*,
                                   float*, float*, float*, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                                   int64_t, float, float, float, void*) {
  return dsa::set_error(DSA_ERR_UNSUPPORTED, "dsa_indexer_kl_grad: not built yet");
}
extern "C" int dsa_compressor_fwd(const float*, const float*, const float*, const float*, void*, int, int64_t,
                                  int64_t, int64_t, int64_t, int, float, void*) {
  return dsa::set_error(DSA_ERR_UNSUPPORTED, "dsa_compressor_fwd: not built yet");
}
