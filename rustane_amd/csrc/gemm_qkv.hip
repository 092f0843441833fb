// Prefill QKV projection (RoPE, head-major Q/K, V and V^T epilogue).
#include "gemm_launch.hpp"

namespace hb {

hipError_t gemm_qkv(const f16* W, const f16* X, int N, int T, int K, const EpiQKV& e,
                    hipStream_t st, int kw) {
  if (e.S < 1 || e.hd < 1 || e.d_pos) return hipErrorInvalidValue;  // prefill: positions from t
  auto run = [&](auto mode) {
    EpiQKVAt<false, decltype(mode)::value> ep(e);
    ep.prepare();
    return launch_gemm(W, X, N, T, K, ep, nullptr, st, {}, kw);
  };
  switch (e.mode()) {
    case EpiQKV::PLAIN: return run(std::integral_constant<int, EpiQKV::PLAIN>{});
    case EpiQKV::SPLIT: return run(std::integral_constant<int, EpiQKV::SPLIT>{});
    default: return run(std::integral_constant<int, EpiQKV::FULL>{});
  }
}

}  // namespace hb
