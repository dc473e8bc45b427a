// Causal depthwise short conv + SiLU for the Gated DeltaNet mixer (gfx950).
//
// Two kernels:
//  * conv_fork_kernel: both streams of the state fork in one pass. Activations are token-major
//    [B, L, conv_dim] (the projection output layout), so a wavefront covers consecutive channels of
//    one token and every global access is a contiguous, vectorised row segment; each thread walks
//    the 32 positions of one block with the last K-1 inputs held in registers, so every input is
//    read once. The noised stream of block k starts from the clean stream's last K-1 pre-conv
//    values before the block (the conv-prefix carry-in); those values are also written out as the
//    fork's conv tails [B*nb, conv_dim, K-1].
//  * conv_generic_kernel: the drop-in causal_conv1d over an arbitrary-strided [B, C, T] input with
//    an optional [B, C, P] prefix, writing token-major output.
//
// Arithmetic follows the reference cast points: the input is converted to the weight's dtype, the
// K products are accumulated in fp32, the sum is rounded to the weight dtype, SiLU is evaluated in
// fp32 (hardware exp2 and reciprocal) and rounded to the weight dtype, and the result is returned
// in the input dtype.
#include "common.h"

namespace dllm {

template <typename T, int N> struct alignas(sizeof(T) * N) VecN { T v[N]; };

// BLK > 0 fixes the block length at compile time: the row loop unrolls completely and the K-1-row
// history stays in registers without moves between rows.
template <typename TX, typename TW, int K, int VEC, int BLK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BLK > 0 ? 5 : 1, BLK > 0 ? 5 : 8))) void conv_fork_kernel(
    const TX* __restrict__ raw0, const TX* __restrict__ rawt, const TW* __restrict__ w,
    const TW* __restrict__ bias, TX* __restrict__ y0, TX* __restrict__ yt, TX* __restrict__ tails,
    int L, int Cd, int block, int cold_noised, int kb_off, int cy) {
  const int cg = blockIdx.x * blockDim.x + threadIdx.x;  // channel group
  const int c0 = cg * VEC;
  if (c0 >= cy) return;  // channels [cy, Cd): not this launch's (their conv runs elsewhere)
  if (BLK > 0) block = BLK;
  const int kblk = blockIdx.y + kb_off;  // the launch covers blocks [kb_off, kb_off + gridDim.y)
  const int b = blockIdx.z;
  const int nb = L / block;

  float wv[VEC][K];
  float bv[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
#pragma unroll
    for (int j = 0; j < K; ++j) wv[e][j] = to_f32(w[(long long)(c0 + e) * K + j]);
    bv[e] = bias ? to_f32(bias[c0 + e]) : 0.f;
  }

  const long long row_base = (long long)b * L * Cd;
  // clean prefix: raw0 positions kblk*block-(K-1)+j, zero before the sequence start
  float h0[K - 1][VEC], ht[K - 1][VEC];
  TX tl[VEC * (K - 1)];  // this thread's conv tails, channel-major: VEC*(K-1) consecutive elements
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const int p = fork_prefix_pos(kblk, j, block, K);
    TX xs[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) xs[e] = from_f32<TX>(0.f);
    if (p >= 0) {
      const TX* src = raw0 + row_base + (long long)p * Cd + c0;
#pragma unroll
      for (int e = 0; e < VEC; ++e) xs[e] = src[e];
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      tl[e * (K - 1) + j] = xs[e];
      h0[j][e] = round_through<TW>(to_f32(xs[e]));
      ht[j][e] = cold_noised ? 0.f : h0[j][e];
    }
  }
  if (tails) {
    TX* dst = tails + ((long long)fork_row(b, kblk, nb) * Cd + c0) * (K - 1);
    constexpr int TN = VEC * (K - 1);
    // widest store dividing the run: the run starts at element c0 * (K - 1), c0 a multiple of VEC
    constexpr int TB = TN * (int)sizeof(TX);
    constexpr int SB = TB % 16 == 0 ? 16 : TB % 8 == 0 ? 8 : 0;
    if constexpr (SB > 0) {
      constexpr int EPS = SB / (int)sizeof(TX);
      typedef VecN<TX, EPS> Vst;
#pragma unroll
      for (int i = 0; i < TN / EPS; ++i) {
        Vst v;
#pragma unroll
        for (int e = 0; e < EPS; ++e) v.v[e] = tl[i * EPS + e];
        *(Vst*)(dst + i * EPS) = v;
      }
    } else {
#pragma unroll
      for (int i = 0; i < TN; ++i) dst[i] = tl[i];
    }
  }

  // rows in groups of RG: the group's loads are issued together before any of its rows is
  // computed, so each thread keeps 2*RG row loads in flight
  constexpr int RG = 4;
  const long long base = row_base + (long long)(kblk * block) * Cd + c0;
  for (int r0 = 0; r0 < block; r0 += RG) {
    VecN<TX, VEC> x0v[RG], xtv[RG];
#pragma unroll
    for (int q = 0; q < RG; ++q) {
      const int r = min(r0 + q, block - 1);  // a ragged last group reloads the last row, unused
      x0v[q] = *(const VecN<TX, VEC>*)(raw0 + base + (long long)r * Cd);
      xtv[q] = *(const VecN<TX, VEC>*)(rawt + base + (long long)r * Cd);
    }
#pragma unroll
    for (int q = 0; q < RG; ++q) {
      if (r0 + q >= block) break;
      const TX* x0 = x0v[q].v;
      const TX* xt = xtv[q].v;
      VecN<TX, VEC> o0v, otv;
      TX* o0 = o0v.v;
      TX* ot = otv.v;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float c0v = round_through<TW>(to_f32(x0[e]));
        const float ctv = round_through<TW>(to_f32(xt[e]));
        float a0 = bv[e], at = bv[e];
#pragma unroll
        for (int j = 0; j < K - 1; ++j) {
          a0 = __builtin_fmaf(wv[e][j], h0[j][e], a0);
          at = __builtin_fmaf(wv[e][j], ht[j][e], at);
        }
        a0 = __builtin_fmaf(wv[e][K - 1], c0v, a0);
        at = __builtin_fmaf(wv[e][K - 1], ctv, at);
        a0 = round_through<TW>(a0);
        at = round_through<TW>(at);
        o0[e] = from_f32<TX>(round_through<TW>(silu_f32(a0)));
        ot[e] = from_f32<TX>(round_through<TW>(silu_f32(at)));
#pragma unroll
        for (int j = 0; j < K - 2; ++j) { h0[j][e] = h0[j + 1][e]; ht[j][e] = ht[j + 1][e]; }
        h0[K - 2][e] = c0v;
        ht[K - 2][e] = ctv;
      }
      const long long off = base + (long long)(r0 + q) * Cd;
      *(VecN<TX, VEC>*)(y0 + off) = o0v;
      *(VecN<TX, VEC>*)(yt + off) = otv;
    }
  }
}

// Generic strided conv: thread = one channel x one segment of SEG positions.
template <typename TX, typename TW>
__global__ __launch_bounds__(256) void conv_generic_kernel(
    const TX* __restrict__ x, long long sxb, long long sxc, long long sxt,
    const TX* __restrict__ pre, long long spb, long long spc, long long spt, int P,
    const TW* __restrict__ w, const TW* __restrict__ bias, TX* __restrict__ y,
    int C, int T, int K, int seg, int silu) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  const int t_begin = blockIdx.y * seg;
  const int b = blockIdx.z;
  const int t_end = min(T, t_begin + seg);
  float wv[8];
  for (int j = 0; j < K; ++j) wv[j] = to_f32(w[(long long)c * K + j]);
  const float bv = bias ? to_f32(bias[c]) : 0.f;
  auto at = [&](int e) -> float {  // extended position e relative to x's first position
    if (e >= 0) return round_through<TW>(to_f32(x[b * sxb + c * sxc + (long long)e * sxt]));
    if (e >= -P) return round_through<TW>(to_f32(pre[b * spb + c * spc + (long long)(P + e) * spt]));
    return 0.f;
  };
  for (int t = t_begin; t < t_end; ++t) {
    float a = bv;
    for (int j = 0; j < K; ++j) a = __builtin_fmaf(wv[j], at(t - (K - 1) + j), a);
    a = round_through<TW>(a);
    if (silu) a = round_through<TW>(silu_f32(a));
    y[((long long)b * T + t) * C + c] = from_f32<TX>(a);
  }
}

template <typename TX, typename TW>
static int launch_fork(const void* raw0, const void* rawt, const void* w, const void* bias, void* y0,
                       void* yt, void* tails, int B, int L, int Cd, int K, int block, int cold, int kb0,
                       int nkb, int cy, hipStream_t st) {
  const int nb = nkb;  // blocks of this launch, from kb0
  constexpr int V = 16 / sizeof(TX);  // 16-byte row segments per thread
  const bool vec_ok = (Cd % V == 0) && (cy % V == 0) && ((uintptr_t)raw0 % 16 == 0) && ((uintptr_t)rawt % 16 == 0) &&
                      ((uintptr_t)y0 % 16 == 0) && ((uintptr_t)yt % 16 == 0) &&
                      ((uintptr_t)tails % 16 == 0);  // tails rows of VEC*(K-1) elements are 16-byte multiples
  bool done = false;
  if constexpr (V == 8) {
    if (K == 4 && vec_ok && block == 32) {
      // 8-byte channel groups at five resident waves per SIMD: at the 27B-class shape (B = 4,
      // L = 4096, conv_dim = 10240) the 20480 waves are exactly four rounds of the chip's slots
      const int groups = cy / 4;
      dim3 grid((groups + 255) / 256, nb, B);
      conv_fork_kernel<TX, TW, 4, 4, 32><<<grid, 256, 0, st>>>(
          (const TX*)raw0, (const TX*)rawt, (const TW*)w, (const TW*)bias, (TX*)y0, (TX*)yt, (TX*)tails, L,
          Cd, block, cold, kb0, cy);
      done = true;
    }
  }
  if (done) {
  } else if (K == 4 && vec_ok) {
    const int groups = cy / V;
    dim3 grid((groups + 255) / 256, nb, B);
    conv_fork_kernel<TX, TW, 4, V, 0><<<grid, 256, 0, st>>>(
        (const TX*)raw0, (const TX*)rawt, (const TW*)w, (const TW*)bias, (TX*)y0, (TX*)yt, (TX*)tails, L,
        Cd, block, cold, kb0, cy);
  } else if (K == 4) {
    dim3 grid((cy + 255) / 256, nb, B);
    conv_fork_kernel<TX, TW, 4, 1, 0><<<grid, 256, 0, st>>>(
        (const TX*)raw0, (const TX*)rawt, (const TW*)w, (const TW*)bias, (TX*)y0, (TX*)yt, (TX*)tails, L,
        Cd, block, cold, kb0, cy);
  } else if (K == 2) {
    dim3 grid((cy + 255) / 256, nb, B);
    conv_fork_kernel<TX, TW, 2, 1, 0><<<grid, 256, 0, st>>>(
        (const TX*)raw0, (const TX*)rawt, (const TW*)w, (const TW*)bias, (TX*)y0, (TX*)yt, (TX*)tails, L,
        Cd, block, cold, kb0, cy);
  } else if (K == 3) {
    dim3 grid((cy + 255) / 256, nb, B);
    conv_fork_kernel<TX, TW, 3, 1, 0><<<grid, 256, 0, st>>>(
        (const TX*)raw0, (const TX*)rawt, (const TW*)w, (const TW*)bias, (TX*)y0, (TX*)yt, (TX*)tails, L,
        Cd, block, cold, kb0, cy);
  } else {
    return fail(DLLM_EUNSUPPORTED, "conv fork: kernel width %d not supported (2, 3 or 4)", K);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "conv fork launch: %s", hipGetErrorString(e));
  return DLLM_OK;
}

}  // namespace dllm

using namespace dllm;

// The fork conv over blocks [kb0, kb1) of every sequence.
static int conv_fork(const void* raw0, const void* rawt, const void* weight, const void* bias, void* y0, void* yt,
                     void* tails, int B, int L, int conv_dim, int width, int block, int dtype_x, int dtype_w,
                     int flags, int kb0, int kb1, hipStream_t st, int y_channels = -1) {
  if (!raw0 || !rawt || !weight || !y0 || !yt) return fail(DLLM_EINVAL, "conv fork: null pointer");
  if (B <= 0 || L <= 0 || conv_dim <= 0 || block <= 0)
    return fail(DLLM_EINVAL, "conv fork: bad sizes B=%d L=%d conv_dim=%d block=%d", B, L, conv_dim, block);
  if (L % block) return fail(DLLM_EINVAL, "L=%d is not a multiple of block=%d", L, block);
  if (L / block > 65535 || B > 65535) return fail(DLLM_EUNSUPPORTED, "conv fork: grid too large");
  if (kb0 < 0 || kb1 > L / block || kb0 >= kb1)
    return fail(DLLM_EINVAL, "conv fork: block range [%d, %d) of %d", kb0, kb1, L / block);
  const int cold = flags & 1, n = kb1 - kb0;
  const int cy = y_channels < 0 ? conv_dim : y_channels;
  if (cy > conv_dim) return fail(DLLM_EINVAL, "conv fork: y_channels %d > conv_dim %d", cy, conv_dim);
  if (cy == 0) return DLLM_OK;
  if (dtype_x == DT_BF16 && dtype_w == DT_BF16)
    return launch_fork<bf16, bf16>(raw0, rawt, weight, bias, y0, yt, tails, B, L, conv_dim, width, block, cold, kb0, n, cy, st);
  if (dtype_x == DT_F32 && dtype_w == DT_F32)
    return launch_fork<float, float>(raw0, rawt, weight, bias, y0, yt, tails, B, L, conv_dim, width, block, cold, kb0, n, cy, st);
  if (dtype_x == DT_BF16 && dtype_w == DT_F32)
    return launch_fork<bf16, float>(raw0, rawt, weight, bias, y0, yt, tails, B, L, conv_dim, width, block, cold, kb0, n, cy, st);
  if (dtype_x == DT_F32 && dtype_w == DT_BF16)
    return launch_fork<float, bf16>(raw0, rawt, weight, bias, y0, yt, tails, B, L, conv_dim, width, block, cold, kb0, n, cy, st);
  return fail(DLLM_EUNSUPPORTED, "conv fork: dtype pair (%d, %d) not supported", dtype_x, dtype_w);
}

extern "C" int dllm_conv_fork_fwd(const void* raw0, const void* rawt, const void* weight, const void* bias,
                                  void* y0, void* yt, void* tails, int B, int L, int conv_dim, int width,
                                  int block, int dtype_x, int dtype_w, int flags, void* stream) {
  const int nb = block > 0 && L > 0 && L % block == 0 ? L / block : 1;  // sizes are checked by conv_fork
  return conv_fork(raw0, rawt, weight, bias, y0, yt, tails, B, L, conv_dim, width, block, dtype_x, dtype_w, flags, 0,
                   nb, (hipStream_t)stream);
}

extern "C" int dllm_conv_fork_channels_range_fwd(const void* raw0, const void* rawt, const void* weight,
                                                 const void* bias, void* y0, void* yt, void* tails, int B, int L,
                                                 int conv_dim, int width, int block, int dtype_x, int dtype_w,
                                                 int flags, int block_begin, int block_end, int y_channels,
                                                 void* stream) {
  if (y_channels < 0) return fail(DLLM_EINVAL, "conv fork: y_channels %d < 0", y_channels);
  return conv_fork(raw0, rawt, weight, bias, y0, yt, tails, B, L, conv_dim, width, block, dtype_x, dtype_w, flags,
                   block_begin, block_end, (hipStream_t)stream, y_channels);
}

extern "C" int dllm_conv_fork_range_fwd(const void* raw0, const void* rawt, const void* weight, const void* bias,
                                        void* y0, void* yt, void* tails, int B, int L, int conv_dim, int width,
                                        int block, int dtype_x, int dtype_w, int flags, int block_begin,
                                        int block_end, void* stream) {
  return conv_fork(raw0, rawt, weight, bias, y0, yt, tails, B, L, conv_dim, width, block, dtype_x, dtype_w, flags,
                   block_begin, block_end, (hipStream_t)stream);
}

extern "C" int dllm_causal_conv1d_fwd(const void* x, const int64_t* x_strides, const void* prefix,
                                      const int64_t* prefix_strides, int prefix_len, const void* weight,
                                      const void* bias, void* y, int B, int C, int T, int width, int dtype_x,
                                      int dtype_w, int activation, void* stream) {
  if (!x || !x_strides || !weight || !y) return fail(DLLM_EINVAL, "causal_conv1d: null pointer");
  if (B <= 0 || C <= 0 || T <= 0 || width <= 0 || width > 8)
    return fail(DLLM_EINVAL, "causal_conv1d: bad sizes B=%d C=%d T=%d K=%d", B, C, T, width);
  if (prefix_len < 0 || (prefix_len > 0 && (!prefix || !prefix_strides)))
    return fail(DLLM_EINVAL, "causal_conv1d: bad prefix");
  // positions per thread: halved until the grid has enough workgroups to fill the chip, so a short
  // segment (a decoding step of one block) still spreads over every CU
  int seg = 64;
  while (seg > 1 && (long long)((C + 255) / 256) * B * ((T + seg - 1) / seg) < 2048) seg >>= 1;
  dim3 grid((C + 255) / 256, (T + seg - 1) / seg, B);
  if (grid.y > 65535 || grid.z > 65535) return fail(DLLM_EUNSUPPORTED, "causal_conv1d: grid too large");
  hipStream_t st = (hipStream_t)stream;
  const long long* ps = (const long long*)prefix_strides;
  const long long* xs = (const long long*)x_strides;
  long long p0 = prefix_len ? ps[0] : 0, p1 = prefix_len ? ps[1] : 0, p2 = prefix_len ? ps[2] : 0;
#define CONV_GENERIC(TX, TW)                                                                           \
  conv_generic_kernel<TX, TW><<<grid, 256, 0, st>>>((const TX*)x, xs[0], xs[1], xs[2], (const TX*)prefix, \
                                                     p0, p1, p2, prefix_len, (const TW*)weight,          \
                                                     (const TW*)bias, (TX*)y, C, T, width, seg, activation)
  if (dtype_x == DT_BF16 && dtype_w == DT_BF16) CONV_GENERIC(bf16, bf16);
  else if (dtype_x == DT_F32 && dtype_w == DT_F32) CONV_GENERIC(float, float);
  else if (dtype_x == DT_BF16 && dtype_w == DT_F32) CONV_GENERIC(bf16, float);
  else if (dtype_x == DT_F32 && dtype_w == DT_BF16) CONV_GENERIC(float, bf16);
  else return fail(DLLM_EUNSUPPORTED, "causal_conv1d: dtype pair (%d, %d) not supported", dtype_x, dtype_w);
#undef CONV_GENERIC
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "causal_conv1d launch: %s", hipGetErrorString(e));
  return DLLM_OK;
}
