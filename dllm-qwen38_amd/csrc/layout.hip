// Integer fork layout of the state fork, produced on the device by the same index functions the
// conv kernel uses (fork_row / fork_state_src / fork_prefix_pos), so that it can be compared
// bit-exactly with the reference's tensor construction.
#include "common.h"

namespace dllm {

__global__ void fork_layout_kernel(int B, int nb, int block, int width, int32_t* row, int32_t* src,
                                   int32_t* pre) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * nb) return;
  const int b = i / nb, k = i % nb;
  const int r = fork_row(b, k, nb);
  row[i] = r;
  src[r] = fork_state_src(b, k, nb);
  for (int j = 0; j < width - 1; ++j) pre[(long long)r * (width - 1) + j] = fork_prefix_pos(k, j, block, width);
}

}  // namespace dllm

using namespace dllm;

extern "C" int dllm_fork_layout(int B, int L, int block, int width, int32_t* row, int32_t* state_src,
                                int32_t* prefix_pos, void* stream) {
  if (!row || !state_src || (!prefix_pos && width > 1)) return fail(DLLM_EINVAL, "fork layout: null pointer");
  if (B <= 0 || L <= 0 || block <= 0 || width < 1) return fail(DLLM_EINVAL, "fork layout: bad sizes");
  if (L % block) return fail(DLLM_EINVAL, "L=%d is not a multiple of block=%d", L, block);
  const int nb = L / block;
  if ((long long)B * nb > 0x7fffffffLL) return fail(DLLM_EUNSUPPORTED, "fork layout: %d x %d fork rows", B, nb);
  const int n = B * nb;
  fork_layout_kernel<<<(n + 255) / 256, 256, 0, (hipStream_t)stream>>>(B, nb, block, width, row, state_src,
                                                                       prefix_pos);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "fork layout launch: %s", hipGetErrorString(e));
  return DLLM_OK;
}
