// Stage 1 MFMA score kernel (bf16). Placeholder: score_mfma_supported()
// returns false so every call takes the exact FP64 kernel.
#include "score_mfma.hpp"

namespace msa {

bool score_mfma_supported(int, int) { return false; }

int score_fwd_mfma_launch(const void*, const void*, const int32_t*, int, int64_t, int, int, int, int, double, float*,
                          int32_t*, hipStream_t) {
  return kErrUnsupported;
}

}  // namespace msa
