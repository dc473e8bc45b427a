// Projections of a decoding step: y[M, N] = x[M, K] W[N, K]^T with few token rows (M <= 64), bf16
// in and out, fp32 accumulation (gfx950).
//
// A cached denoising step runs every projection of the stack on one block of tokens (32 rows), so
// each weight is read once for 32 rows and the step is bound by streaming the weights from HBM.
// The library GEMMs stream the wide projections well, but a narrow one (the per-head gates, the
// attention k and v: N <= 2048) costs them a fixed ~19 us, and a deep one (the MLP down
// projection, K = 17408) runs at ~2.2 TB/s; this kernel takes those. The weights stream straight
// into MFMA operands:
//   * a workgroup owns 32 output features (one 32x32 accumulator tile) and a range of K; its four
//     waves split that range; per step of 64 k a lane loads 64 contiguous bytes of one weight row
//     (B operand, lane = feature) and of one token row (A operand, lane = token; the token rows
//     are small and stay in L2), and issues four v_mfma_f32_32x32x16_bf16. Lane (row, h) carries
//     k = 32h + 8u + 0..7 in MFMA u for both operands, so the contraction is exact in any order;
//   * the four waves' tiles are summed through LDS in a fixed order; with one K range the sum is
//     rounded to bf16 and stored, otherwise fp32 partials [S, M, N] go to a workspace and a second
//     kernel sums them in split order. Results are deterministic run to run.
//   * more than 32 token rows: grid.z takes the next 32 rows (the weights are streamed again).
#include "common.h"

namespace dllm {

constexpr int LIN_UNROLL = 2;  // 64-k steps per loop iteration: 8 x 16-byte loads in flight per operand

__global__ __launch_bounds__(256) void decode_linear_kernel(const bf16* __restrict__ x, const bf16* __restrict__ w,
                                                           bf16* __restrict__ y, float* __restrict__ part, int M, int N,
                                                           int K, int kchunk) {
  __shared__ __attribute__((aligned(16))) float red[4][16][64];  // [wave][value][lane]
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int tile = blockIdx.x, split = blockIdx.y, m0 = blockIdx.z * 32;
  const int n = tile * 32 + l32;
  const int m = m0 + l32;
  const bool nok = n < N, mok = m < M;
  const bf16* wr = w + (long long)(nok ? n : N - 1) * K;
  const bf16* xr = x + (long long)(mok ? m : 0) * K;
  const int kq = kchunk / 4;                       // this wave's share, a multiple of 64
  const int kb = split * kchunk + wave * kq;
  const int ke = min(K, kb + kq);
  f32x16 acc = zero16();
  const bf16x8 z8 = {};
  int k0 = kb;
  for (; k0 + 64 * LIN_UNROLL <= ke; k0 += 64 * LIN_UNROLL) {
    bf16x8 wv[LIN_UNROLL][4], xv[LIN_UNROLL][4];
#pragma unroll
    for (int s = 0; s < LIN_UNROLL; ++s)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        wv[s][u] = *(const bf16x8*)(wr + k0 + 64 * s + 32 * h + 8 * u);
        xv[s][u] = mok ? *(const bf16x8*)(xr + k0 + 64 * s + 32 * h + 8 * u) : z8;
      }
#pragma unroll
    for (int s = 0; s < LIN_UNROLL; ++s)
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xv[s][u], wv[s][u], acc, 0, 0, 0);
  }
  for (; k0 < ke; k0 += 64) {  // K is a multiple of 64
    bf16x8 wv[4], xv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      wv[u] = *(const bf16x8*)(wr + k0 + 32 * h + 8 * u);
      xv[u] = mok ? *(const bf16x8*)(xr + k0 + 32 * h + 8 * u) : z8;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xv[u], wv[u], acc, 0, 0, 0);
  }
  // acc: lane holds feature column l32, token rows rho(v, h); sum the four waves in wave order
#pragma unroll
  for (int v = 0; v < 16; ++v) red[wave][v][lane] = acc[v];
  __syncthreads();
  // thread -> (lane ln, values 4g .. 4g+3): token rows 8g + 4hh + 0..3, feature ln % 32
  const int ln = tid & 63, g = tid >> 6, hh = ln >> 5;
  const int nn = tile * 32 + (ln & 31);
  if (nn >= N) return;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int v = 4 * g + e;
    const float sum = ((red[0][v][ln] + red[1][v][ln]) + red[2][v][ln]) + red[3][v][ln];
    const int mm = m0 + 8 * g + 4 * hh + e;
    if (mm >= M) continue;
    if (part) part[((long long)split * M + mm) * N + nn] = sum;
    else y[(long long)mm * N + nn] = (bf16)sum;
  }
}

// y = bf16(sum over splits of part[s]) in split order
__global__ __launch_bounds__(256) void decode_linear_reduce_kernel(const float* __restrict__ part, bf16* __restrict__ y,
                                                                  long long MN, int S) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= MN) return;
  float s = part[i];
  for (int j = 1; j < S; ++j) s += part[(long long)j * MN + i];
  y[i] = (bf16)s;
}

}  // namespace dllm

using namespace dllm;

extern "C" int dllm_decode_linear_splits(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64) return 0;
  const long long tiles = (long long)((N + 31) / 32) * ((M + 31) / 32);
  // about two workgroups per CU, each K range at least 256 deep and at most 8 splits (measured: more
  // splits cost more in partial sums than they gain in parallelism)
  long long s = (512 + tiles - 1) / tiles;
  long long smax = K / 256 > 0 ? K / 256 : 1;
  if (smax > 8) smax = 8;
  if (s > smax) s = smax;
  if (s < 1) s = 1;
  return (int)s;
}

extern "C" int dllm_decode_linear_fwd(const void* x, const void* weight, void* y, float* workspace, int M, int N, int K,
                                      int splits, int dtype, void* stream) {
  if (!x || !weight || !y) return fail(DLLM_EINVAL, "decode linear: null pointer");
  if (M <= 0 || N <= 0 || K <= 0 || splits <= 0) return fail(DLLM_EINVAL, "decode linear: bad sizes M=%d N=%d K=%d", M, N, K);
  if (dtype != DT_BF16) return fail(DLLM_EUNSUPPORTED, "decode linear: bf16 only");
  if (K % 64) return fail(DLLM_EUNSUPPORTED, "decode linear: K=%d is not a multiple of 64", K);
  if (M > 64) return fail(DLLM_EUNSUPPORTED, "decode linear: M=%d > 64 rows (use a library GEMM)", M);
  if (((uintptr_t)x | (uintptr_t)weight) & 15) return fail(DLLM_EINVAL, "decode linear: x and weight must be 16-byte aligned");
  if (splits > 1 && !workspace) return fail(DLLM_EINVAL, "decode linear: %d splits need a workspace", splits);
  // K range per split: a multiple of 256 (four waves of 64-k steps)
  const int kchunk = ((K + splits - 1) / splits + 255) / 256 * 256;
  const int S = (K + kchunk - 1) / kchunk;
  const unsigned tiles = (unsigned)((N + 31) / 32);
  if (tiles > 0x7fffffffu) return fail(DLLM_EUNSUPPORTED, "decode linear: grid too large");
  hipStream_t st = (hipStream_t)stream;
  decode_linear_kernel<<<dim3(tiles, S, (M + 31) / 32), 256, 0, st>>>(
      (const bf16*)x, (const bf16*)weight, (bf16*)y, S > 1 ? workspace : nullptr, M, N, K, kchunk);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "decode linear launch: %s", hipGetErrorString(e));
  if (S > 1) {
    const long long MN = (long long)M * N;
    decode_linear_reduce_kernel<<<dim3((unsigned)((MN + 255) / 256)), 256, 0, st>>>(workspace, (bf16*)y, MN, S);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(DLLM_ELAUNCH, "decode linear reduce launch: %s", hipGetErrorString(e));
  }
  return DLLM_OK;
}
