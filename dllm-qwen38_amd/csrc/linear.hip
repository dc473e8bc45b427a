// Projections of a decoding step: y[M, N] = x[M, K] W[N, K]^T with few token rows (M <= 64), bf16
// in and out, fp32 accumulation (gfx950).
//
// A cached denoising step runs every projection of the stack on one block of tokens (32 rows), so
// each weight is read once for 32 rows and the step is bound by streaming the weights from HBM.
// The weights stream through LDS in wide coalesced reads:
//   * a workgroup owns 128 output features (four 32x32 accumulator tiles, one per wave) and a
//     range of K. Per step of 64 k it stages the weight tile [128 features x 64 k] and the token
//     tile [32 rows x 64 k] with direct global -> LDS loads (each wave instruction moves 1 KB: eight
//     whole 128-byte row segments, no registers), in a ring of LIN_NST stages that keeps
//     LIN_NST - 1 steps in flight;
//   * rows are 128 bytes with their 16-byte chunks XOR-swizzled by (row >> 1), so the operand reads
//     (16 rows of one chunk per pass) touch every bank once;
//   * wave w reads the B operand (lane = feature) of its 32 features and the A operand (lane =
//     token) from LDS, 16 bytes each, and issues four v_mfma_f32_32x32x16_bf16 per step (lane
//     (row, h) carries k = 16u + 8h + 0..7 in MFMA u for both operands);
//   * with one K range the tile is rounded to bf16 and stored; with several, fp32 partials
//     [S, M, N] go to a workspace and a second kernel sums them in split order (deterministic);
//   * more than 32 token rows: grid.z takes the next 32 rows (the weights are streamed again);
//   * up to four projections of the same x (q | k | v, the four mixer inputs, gate | up) share one
//     launch and one split reduction: the grid's tiles run through the weights in turn. With the
//     SwiGLU epilogue (gate | up) the reduction writes round(round(silu(gate)) * up), the MLP's
//     activation, instead of the two projections.
#include "common.h"

namespace dllm {

constexpr int LIN_NST = 3;                 // ring stages
constexpr int LIN_W_BYTES = 128 * 64 * 2;  // weight tile of one step
constexpr int LIN_X_BYTES = 32 * 64 * 2;   // token tile of one step
constexpr int LIN_STAGE = LIN_W_BYTES + LIN_X_BYTES;

__device__ __forceinline__ int lin_off(int row, int chunk) {  // byte offset of a 16-byte chunk of a 128-byte row
  return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4);
}

template <int N>
__device__ __forceinline__ void lin_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

constexpr int LIN_MAXSEG = 4;
struct LinSeg {
  const bf16* w;  // [N, K]
  bf16* y;        // [M, N]
  float* part;    // [S, M, N] fp32 partials (split path)
  int N;
  int tile0;      // first grid tile of this projection
  long long e0;   // first element of this projection in the reduction's index space
};
struct LinArgs {
  const bf16* x;
  LinSeg seg[LIN_MAXSEG];
  int nseg, M, K, kchunk, S, split_path, swiglu;
};

__global__ __launch_bounds__(256) void decode_linear_kernel(LinArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[LIN_NST * LIN_STAGE];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int split = blockIdx.y, m0 = blockIdx.z * 32;
  int si = 0;
#pragma unroll
  for (int i = 1; i < LIN_MAXSEG; ++i)
    if (i < a.nseg && (int)blockIdx.x >= a.seg[i].tile0) si = i;
  const LinSeg& sg = a.seg[si];
  const bf16* __restrict__ const x = a.x;
  const bf16* __restrict__ const w = sg.w;
  const int M = a.M, N = sg.N, K = a.K, kchunk = a.kchunk;
  const int tile = blockIdx.x - sg.tile0;
  const int n0 = tile * 128;
  const int kb = split * kchunk;
  const int ke = min(K, kb + kchunk);
  const int nsteps = ke > kb ? (ke - kb) / 64 : 0;  // K and kchunk are multiples of 64

  // staging role of this lane: row 8 i + lane / 8 of its rows, logical chunk (lane % 8) ^ key(row)
  const int srow = lane >> 3, schunk = lane & 7;
  auto stage = [&](int s) {
    unsigned char* sb = smem + (s % LIN_NST) * LIN_STAGE;
    const int k0 = kb + 64 * s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // this wave's 4 of the 16 weight instructions: rows 32 wave + 8 i ..
      const int row = 32 * wave + 8 * i + srow;
      const int n = min(n0 + row, N - 1);  // rows past N load a valid row; their outputs are not stored
      const int c = schunk ^ ((row >> 1) & 7);
      const bf16* src = w + (long long)n * K + k0 + 8 * c;
      dma_load16(src, sb + (32 * wave + 8 * i) * 128);
    }
    {  // token tile: wave w stages rows 8 w .. 8 w + 7
      const int row = 8 * wave + srow;
      const int m = min(m0 + row, M - 1);
      const int c = schunk ^ ((row >> 1) & 7);
      const bf16* src = x + (long long)m * K + k0 + 8 * c;
      dma_load16(src, sb + LIN_W_BYTES + 8 * wave * 128);
    }
  };
  constexpr int PER = 5;  // direct loads per wave per step
  static_assert(LIN_NST == 3, "wait_step assumes at most one step in flight behind the waited one");
  auto wait_step = [&](int s) {  // step s has landed for this wave (step s + 1 may still travel)
    if (s + 1 < nsteps) lin_wait_vmcnt<PER>();
    else lin_wait_vmcnt<0>();
  };

  f32x16 acc = zero16();
#pragma unroll
  for (int s = 0; s < LIN_NST - 1; ++s)
    if (s < nsteps) stage(s);
  if (nsteps > 0) wait_step(0);
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    if (s + LIN_NST - 1 < nsteps) stage(s + LIN_NST - 1);  // its stage held step s - 1, done before the barrier
    const unsigned char* sb = smem + (s % LIN_NST) * LIN_STAGE;
    const unsigned char* xs = sb + LIN_W_BYTES;
    bf16x8 a[4], bv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      a[u] = *(const bf16x8*)(xs + lin_off(l32, 2 * u + h));
      bv[u] = *(const bf16x8*)(sb + lin_off(32 * wave + l32, 2 * u + h));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[u], bv[u], acc, 0, 0, 0);
    if (s + 1 < nsteps) wait_step(s + 1);
    __syncthreads();  // step s + 1 staged by every wave; every wave is done with step s's stage
  }
  // acc: lane holds feature column l32 of this wave's tile, token rows rho(v, h)
  const int n = n0 + 32 * wave + l32;
  if (n >= N) return;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int m = m0 + rho(v, h);
    if (m >= M) continue;
    if (a.split_path) sg.part[((long long)split * M + m) * N + n] = acc[v];
    else sg.y[(long long)m * N + n] = (bf16)acc[v];
  }
}

// y = bf16(sum over splits of part[s]) in split order, for every projection of the launch; with
// the SwiGLU epilogue (two projections of equal N) y0 = round(round(silu(gate)) * up) instead.
__global__ __launch_bounds__(256) void decode_linear_reduce_kernel(LinArgs a, long long total) {
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= total) return;
  int si = 0;
#pragma unroll
  for (int i = 1; i < LIN_MAXSEG; ++i)
    if (i < a.nseg && e >= a.seg[i].e0) si = i;
  const long long MN0 = (long long)a.M * a.seg[si].N;
  const long long i = e - a.seg[si].e0;
  const float* p = a.seg[si].part + i;
  float s = p[0];
  for (int j = 1; j < a.S; ++j) s += p[(long long)j * MN0];
  if (!a.swiglu) {
    a.seg[si].y[i] = (bf16)s;
    return;
  }
  const float* pu = a.seg[1].part + i;  // swiglu: index space is the gate's; up has the same shape
  float su = pu[0];
  for (int j = 1; j < a.S; ++j) su += pu[(long long)j * MN0];
  const float g = round_through<bf16>(s), u = round_through<bf16>(su);
  a.seg[0].y[i] = (bf16)(round_through<bf16>(silu_f32(g)) * u);
}

}  // namespace dllm

using namespace dllm;

extern "C" int dllm_decode_linear_splits(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64) return 0;
  const long long tiles = (long long)((N + 127) / 128) * ((M + 31) / 32);
  // about 1.5 workgroups per CU, each K range at least 256 deep and at most 8 splits
  long long s = (384 + tiles - 1) / tiles;
  long long smax = K / 256 > 0 ? K / 256 : 1;
  if (smax > 8) smax = 8;
  if (s > smax) s = smax;
  if (s < 1) s = 1;
  return (int)s;
}

extern "C" int dllm_decode_linear_multi_fwd(const void* x, int M, int K, int count, const void* const* weights,
                                            void* const* outs, const int* Ns, float* workspace, int splits, int swiglu,
                                            int dtype, void* stream) {
  if (!x || !weights || !outs || !Ns) return fail(DLLM_EINVAL, "decode linear: null pointer");
  if (count < 1 || count > LIN_MAXSEG) return fail(DLLM_EINVAL, "decode linear: %d projections (1..%d)", count, LIN_MAXSEG);
  if (M <= 0 || K <= 0 || splits <= 0) return fail(DLLM_EINVAL, "decode linear: bad sizes M=%d K=%d", M, K);
  if (dtype != DT_BF16) return fail(DLLM_EUNSUPPORTED, "decode linear: bf16 only");
  if (K % 64) return fail(DLLM_EUNSUPPORTED, "decode linear: K=%d is not a multiple of 64", K);
  if (M > 64) return fail(DLLM_EUNSUPPORTED, "decode linear: M=%d > 64 rows (use a library GEMM)", M);
  if ((uintptr_t)x & 15) return fail(DLLM_EINVAL, "decode linear: x must be 16-byte aligned");
  if (swiglu && (count != 2 || Ns[0] != Ns[1])) return fail(DLLM_EINVAL, "decode linear: swiglu takes gate | up of equal N");
  LinArgs a = {};
  a.x = (const bf16*)x;
  a.nseg = count;
  a.M = M; a.K = K;
  a.kchunk = ((K + splits - 1) / splits + 63) / 64 * 64;  // K range per split: whole 64-k steps
  a.S = (K + a.kchunk - 1) / a.kchunk;
  a.swiglu = swiglu;
  a.split_path = a.S > 1 || swiglu;
  long long tiles = 0, elems = 0;
  for (int i = 0; i < count; ++i) {
    if (!weights[i] || !outs[i] || Ns[i] <= 0) return fail(DLLM_EINVAL, "decode linear: projection %d is empty", i);
    if ((uintptr_t)weights[i] & 15) return fail(DLLM_EINVAL, "decode linear: weights must be 16-byte aligned");
    LinSeg& sg = a.seg[i];
    sg.w = (const bf16*)weights[i];
    sg.y = (bf16*)outs[i];
    sg.N = Ns[i];
    sg.tile0 = (int)tiles;
    sg.e0 = elems;
    sg.part = a.split_path ? workspace + (long long)a.S * elems : nullptr;
    tiles += (Ns[i] + 127) / 128;
    elems += (long long)M * Ns[i];
  }
  if (a.split_path && !workspace) return fail(DLLM_EINVAL, "decode linear: the split path needs a workspace");
  if (tiles > 0x7fffffffLL) return fail(DLLM_EUNSUPPORTED, "decode linear: grid too large");
  hipStream_t st = (hipStream_t)stream;
  decode_linear_kernel<<<dim3((unsigned)tiles, a.S, (M + 31) / 32), 256, 0, st>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "decode linear launch: %s", hipGetErrorString(e));
  if (a.split_path) {
    const long long total = swiglu ? (long long)M * Ns[0] : elems;
    decode_linear_reduce_kernel<<<dim3((unsigned)((total + 255) / 256)), 256, 0, st>>>(a, total);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(DLLM_ELAUNCH, "decode linear reduce launch: %s", hipGetErrorString(e));
  }
  return DLLM_OK;
}

extern "C" int dllm_decode_linear_fwd(const void* x, const void* weight, void* y, float* workspace, int M, int N, int K,
                                      int splits, int dtype, void* stream) {
  const void* w[1] = {weight};
  void* o[1] = {y};
  const int n[1] = {N};
  return dllm_decode_linear_multi_fwd(x, M, K, 1, w, o, n, workspace, splits, 0, dtype, stream);
}
