// Prefill SwiGLU up-projection and logits GEMMs.
#include "gemm_launch.hpp"

namespace hb {

hipError_t gemm_swiglu(const f16* W, const f16* X, int N, int T, int K, const EpiSwiGLU& e,
                       hipStream_t st, int kw) {
  return launch_gemm(W, X, N, T, K, e, nullptr, st, {}, kw);
}
hipError_t gemm_logits(const f16* W, const f16* X, int N, int T, int K, const EpiLogits& e,
                       hipStream_t st, int kw) {
  return launch_gemm(W, X, N, T, K, e, nullptr, st, {}, kw);
}

}  // namespace hb
