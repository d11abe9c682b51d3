// Stage 3 MFMA kernels (bf16). Placeholder until the MFMA kernels land:
// attn_mfma_supported() returns false so every call takes the VALU path.
#include "attn_mfma.hpp"

namespace msa {

bool attn_mfma_supported(int64_t, int64_t) { return false; }

int attn_fwd_mfma(const void*, const void*, const void*, const int32_t*, const int32_t*, int, int64_t, int, int, int,
                  int, int, float, void*, float*, hipStream_t) {
  return kErrUnsupported;
}

int attn_bwd_dq_mfma(const void*, const void*, const void*, const void*, const void*, const float*, const int32_t*,
                     const int32_t*, int, int64_t, int, int, int, int, int, float, void*, float*, hipStream_t) {
  return kErrUnsupported;
}

int64_t attn_dkdv_mfma_workspace_bytes(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t) { return 256; }

int attn_bwd_dkdv_mfma(const void*, const void*, const void*, const void*, const float*, const float*, const int32_t*,
                       const int32_t*, const int32_t*, const int32_t*, int, int64_t, int, int, int, int64_t, int, float,
                       void*, void*, void*, int64_t, hipStream_t) {
  return kErrUnsupported;
}

}  // namespace msa
