// Backward launch (placeholder until the backward kernels land).
#include "bwd_launch.hpp"
#include "launch.hpp"

namespace af {
size_t bwd_workspace_bytes(int32_t batch, int32_t heads_q, int32_t seqlen_q) {
  if (batch <= 0 || heads_q <= 0 || seqlen_q < 0) return 0;
  return (size_t)batch * heads_q * seqlen_q * sizeof(float);
}
int run_bwd(const af_bwd_args*, const af_blockmask*, void*, size_t, hipStream_t) {
  set_error("backward kernels are not built yet");
  return AF_ERR_UNSUPPORTED;
}
}  // namespace af
