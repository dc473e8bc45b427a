// Row-wise prologue / epilogue kernels around the two mixers (gfx950): the Qwen3.5 RMSNorm with a
// (1 + w) weight (optionally fused with the residual add before it), the gated RMSNorm of the GDN
// output, the SwiGLU product of the MLP, and the attention prologue (per-head q/k RMSNorm followed
// by partial RoPE with positions shared by both halves of cat([x_t, x_0])).
//
// These are HBM-bound: one wave per row, every input read once, fp32 arithmetic, and results
// rounded at the cast points of the transformers modules they replace so that bf16 results match
// them element for element except where a fp32 reduction order differs.
#include "common.h"

namespace dllm {

template <typename T> __device__ __forceinline__ float ld(const T* p) { return to_f32(*p); }

// y = rmsnorm(s) * (1 + w) with s = x (+ r, rounded to T, also written to sum_out)
template <typename T, typename TW, int NV>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const T* __restrict__ x, const T* __restrict__ r,
                                                      T* __restrict__ sum_out, const TW* __restrict__ w,
                                                      T* __restrict__ y, int rows, int dim, float eps, int unit) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const long long base = (long long)row * dim;
  // NV > 0: dim == 64 * 8 * NV, 16-byte vectors; NV == 0: generic strided scalar path
  if constexpr (NV > 0) {
    typedef __attribute__((ext_vector_type(8))) T V8;
    float v[NV][8];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const long long off = base + (long long)(k * 64 + lane) * 8;
      const V8 xv = *(const V8*)(x + off);
      V8 sv = xv;
      if (r) {
        const V8 rv = *(const V8*)(r + off);
#pragma unroll
        for (int i = 0; i < 8; ++i) sv[i] = from_f32<T>(to_f32(xv[i]) + to_f32(rv[i]));
        if (sum_out) *(V8*)(sum_out + off) = sv;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v[k][i] = to_f32(sv[i]);
        ss = __builtin_fmaf(v[k][i], v[k][i], ss);
      }
    }
    const float inv = rsqrtf(wave_sum(ss) / (float)dim + eps);
    typedef __attribute__((ext_vector_type(8))) TW W8;  // weights as vectors too (16 or 32 bytes)
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c0 = (k * 64 + lane) * 8;
      const W8 wv = *(const W8*)(w + c0);
      V8 yv;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float wf = to_f32(wv[i]);
        yv[i] = from_f32<T>(v[k][i] * inv * (unit ? 1.f + wf : wf));
      }
      *(V8*)(y + base + c0) = yv;
    }
  } else {
    float ss = 0.f;
    for (int c = lane; c < dim; c += 64) {
      float s = ld(x + base + c);
      if (r) {
        const T st = from_f32<T>(s + ld(r + base + c));
        if (sum_out) sum_out[base + c] = st;
        s = to_f32(st);
      }
      ss = __builtin_fmaf(s, s, ss);
    }
    const float inv = rsqrtf(wave_sum(ss) / (float)dim + eps);
    for (int c = lane; c < dim; c += 64) {
      const float s = r ? to_f32(from_f32<T>(ld(x + base + c) + ld(r + base + c))) : ld(x + base + c);
      const float wf = to_f32(w[c]);
      y[base + c] = from_f32<T>(s * inv * (unit ? 1.f + wf : wf));
    }
  }
}

// The same for few rows: one workgroup of nw = blockDim.x / 64 waves per row, so that the rows of a
// decoding step (32) spread over 32 CUs instead of 8, with the weights loaded beside the row (before
// the reduction). dim == nw * 512 * NV; lane vectors (k nw + wave) * 64 + lane, 16 bytes each; the
// sum of squares adds the waves' sums in wave order.
template <typename T, typename TW, int NV>
__global__ __launch_bounds__(512) void rmsnorm_row_kernel(const T* __restrict__ x, const T* __restrict__ r,
                                                          T* __restrict__ sum_out, const TW* __restrict__ w,
                                                          T* __restrict__ y, int dim, float eps, int unit) {
  __shared__ float part[8];
  const int nw = blockDim.x >> 6, wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const long long base = (long long)blockIdx.x * dim;
  typedef __attribute__((ext_vector_type(8))) T V8;
  typedef __attribute__((ext_vector_type(8))) TW W8;
  float v[NV][8];
  W8 wt[NV];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c0 = ((k * nw + wv) * 64 + lane) * 8;
    const V8 xv = *(const V8*)(x + base + c0);
    wt[k] = *(const W8*)(w + c0);
    V8 sv = xv;
    if (r) {
      const V8 rv = *(const V8*)(r + base + c0);
#pragma unroll
      for (int i = 0; i < 8; ++i) sv[i] = from_f32<T>(to_f32(xv[i]) + to_f32(rv[i]));
      if (sum_out) *(V8*)(sum_out + base + c0) = sv;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[k][i] = to_f32(sv[i]);
      ss = __builtin_fmaf(v[k][i], v[k][i], ss);
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) part[wv] = ss;
  __syncthreads();
  float tot = part[0];
  for (int i = 1; i < nw; ++i) tot += part[i];
  const float inv = rsqrtf(tot / (float)dim + eps);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c0 = ((k * nw + wv) * 64 + lane) * 8;
    V8 yv;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float wf = to_f32(wt[k][i]);
      yv[i] = from_f32<T>(v[k][i] * inv * (unit ? 1.f + wf : wf));
    }
    *(V8*)(y + base + c0) = yv;
  }
}

// y = (w * round_T(rmsnorm(x))) * silu(z), the product rounded to T at each step as in the module
template <typename T, typename TW>
__global__ __launch_bounds__(256) void gated_rmsnorm_kernel(const T* __restrict__ x, const T* __restrict__ z,
                                                            const TW* __restrict__ w, T* __restrict__ y, int rows,
                                                            int dim, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const long long base = (long long)row * dim;
  float ss = 0.f;
  for (int c = lane; c < dim; c += 64) {
    const float v = ld(x + base + c);
    ss = __builtin_fmaf(v, v, ss);
  }
  const float inv = rsqrtf(wave_sum(ss) / (float)dim + eps);
  for (int c = lane; c < dim; c += 64) {
    const float t = round_through<T>(ld(x + base + c) * inv);
    const float u = round_through<T>(to_f32(w[c]) * t);  // weight (module dtype) * normed (input dtype)
    y[base + c] = from_f32<T>(u * silu_f32(ld(z + base + c)));
  }
}

// The same with 16-byte rows: LPR = dim / 8 lanes per row (dim 64 .. 512), 64 / LPR rows per wave,
// each lane 8 elements of x, z and w; the row's sum of squares by a butterfly over its lanes.
template <int LPR>
__global__ __launch_bounds__(256) void gated_rmsnorm_vec_kernel(const bf16* __restrict__ x, const bf16* __restrict__ z,
                                                                const bf16* __restrict__ w, bf16* __restrict__ y,
                                                                int rows, float eps) {
  constexpr int DIM = 8 * LPR, RPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const long long row = ((long long)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / LPR;
  const int c0 = (lane % LPR) * 8;
  const long long base = (row < rows ? row : rows - 1) * DIM + c0;  // every lane takes part in the butterfly
  const bf16x8 xv = *(const bf16x8*)(x + base), zv = *(const bf16x8*)(z + base), wv = *(const bf16x8*)(w + c0);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = __builtin_fmaf((float)xv[i], (float)xv[i], ss);
#pragma unroll
  for (int off = LPR / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  const float inv = rsqrtf(ss / (float)DIM + eps);
  bf16x8 yv;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float t = round_through<bf16>((float)xv[i] * inv);
    const float u = round_through<bf16>((float)wv[i] * t);
    yv[i] = (bf16)(u * silu_f32((float)zv[i]));
  }
  if (row < rows) *(bf16x8*)(y + base) = yv;
}

// Gated DeltaNet gates of every (token, value head): beta = round_T(sigmoid(b)) held in fp32, and
// g = -exp(A_log) * softplus(a + dt_bias) in fp32 (softplus linear above 20, as torch's).
template <typename T, typename TP>
__global__ __launch_bounds__(256) void gdn_gates_kernel(const T* __restrict__ b, const T* __restrict__ a,
                                                        const TP* __restrict__ a_log, const TP* __restrict__ dt_bias,
                                                        float* __restrict__ beta, float* __restrict__ g, long long n,
                                                        int H) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int h = (int)(i % H);
  const float bv = to_f32(b[i]);
  beta[i] = round_through<T>(1.f / (1.f + expf(-bv)));
  const float av = to_f32(a[i]) + to_f32(dt_bias[h]);
  const float sp = av > 20.f ? av : log1pf(expf(av));
  g[i] = -expf(to_f32(a_log[h])) * sp;
}

// out = round_T(round_T(silu(g)) * u)
template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(const T* __restrict__ g, const T* __restrict__ u,
                                                     T* __restrict__ out, long long n) {
  typedef __attribute__((ext_vector_type(8))) T V8;
  const long long i = ((long long)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i + 8 <= n) {
    const V8 gv = *(const V8*)(g + i), uv = *(const V8*)(u + i);
    V8 o;
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = from_f32<T>(round_through<T>(silu_f32(to_f32(gv[k]))) * to_f32(uv[k]));
    *(V8*)(out + i) = o;
  } else {
    for (long long k = i; k < n; ++k) out[k] = from_f32<T>(round_through<T>(silu_f32(to_f32(g[k]))) * to_f32(u[k]));
  }
}

// Attention prologue: one wave per (token, head) row of q (then k). rmsnorm over the head dim with
// (1 + w), then RoPE on the first rd dims: out = a*cos + rotate_half(a)*sin with every product and
// the sum rounded to T (the module computes them in the activation dtype). Token t of the
// 2L-long sequence uses table row t mod L.
template <typename T, typename TW>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const T* __restrict__ q, long long q_sb, int q_st, int q_sh, const T* __restrict__ k, long long k_sb, int k_st,
    int k_sh, const TW* __restrict__ wq, const TW* __restrict__ wk, const T* __restrict__ cosb,
    const T* __restrict__ sinb, T* __restrict__ qo, T* __restrict__ ko, int B, int S, int L, int Hq, int Hkv, int hd,
    int rd, float eps) {
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const long long nq = (long long)B * S * Hq, nk = (long long)B * S * Hkv;
  if (row >= nq + nk) return;
  const bool isq = row < nq;
  const long long rr = isq ? row : row - nq;
  const int H = isq ? Hq : Hkv;
  const int hh = (int)(rr % H);
  const long long bt = rr / H;
  const int t = (int)(bt % S), b = (int)(bt / S);
  const T* src = isq ? q + b * q_sb + (long long)t * q_st + (long long)hh * q_sh
                     : k + b * k_sb + (long long)t * k_st + (long long)hh * k_sh;
  const TW* w = isq ? wq : wk;
  T* dst = (isq ? qo : ko) + rr * hd;
  constexpr int MAXE = 4;  // hd <= 256
  float v[MAXE];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < MAXE; ++e) {
    const int c = lane + 64 * e;
    v[e] = c < hd ? ld(src + c) : 0.f;
    ss = __builtin_fmaf(v[e], v[e], ss);
  }
  const float inv = rsqrtf(wave_sum(ss) / (float)hd + eps);
  const int pos = t % L;
  const int half = rd / 2;
  // normalised values, rounded to T, then exchanged through the wave for rotate_half
  float nv[MAXE];
#pragma unroll
  for (int e = 0; e < MAXE; ++e) {
    const int c = lane + 64 * e;
    nv[e] = c < hd ? round_through<T>(v[e] * inv * (1.f + to_f32(w[c]))) : 0.f;
  }
#pragma unroll
  for (int e = 0; e < MAXE; ++e) {
    const int c = lane + 64 * e;
    // partner column for rotate_half inside the first rd dims
    const int pc = c < half ? c + half : c - half;
    const int pe = pc >> 6, pl = pc & 63;
    float pv = 0.f;
#pragma unroll
    for (int f = 0; f < MAXE; ++f) {
      const float x = __shfl(nv[f], pl);
      pv = (f == pe) ? x : pv;
    }
    if (c < hd) {
      float o = nv[e];
      if (c < rd) {
        const float cs = to_f32(cosb[(long long)pos * rd + c]), sn = to_f32(sinb[(long long)pos * rd + c]);
        const float rot = c < half ? -pv : pv;
        o = round_through<T>(round_through<T>(nv[e] * cs) + round_through<T>(rot * sn));
      }
      dst[c] = from_f32<T>(o);
    }
  }
}

// The same for bf16 heads of 256 with 8-byte rows: lane l holds columns 4l .. 4l + 3, so the
// rotate_half partner of a rotated column (rd / 2 away) sits in lane l ^ (rd / 8) at the same
// position (rd / 8 a power of two): one lane exchange per element instead of a search over the wave.
__global__ __launch_bounds__(256) void qk_norm_rope256_kernel(
    const bf16* __restrict__ q, long long q_sb, int q_st, int q_sh, const bf16* __restrict__ k, long long k_sb,
    int k_st, int k_sh, const bf16* __restrict__ wq, const bf16* __restrict__ wk, const bf16* __restrict__ cosb,
    const bf16* __restrict__ sinb, bf16* __restrict__ qo, bf16* __restrict__ ko, int B, int S, int L, int Hq, int Hkv,
    int rd, float eps) {
  typedef __attribute__((ext_vector_type(4))) bf16 T4;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const long long nq = (long long)B * S * Hq, nk = (long long)B * S * Hkv;
  if (row >= nq + nk) return;
  const bool isq = row < nq;
  const long long rr = isq ? row : row - nq;
  const int H = isq ? Hq : Hkv;
  const int hh = (int)(rr % H);
  const long long bt = rr / H;
  const int t = (int)(bt % S), b = (int)(bt / S);
  const bf16* src = isq ? q + b * q_sb + (long long)t * q_st + (long long)hh * q_sh
                        : k + b * k_sb + (long long)t * k_st + (long long)hh * k_sh;
  const bf16* w = isq ? wq : wk;
  const int c0 = 4 * lane;
  const T4 xv = *(const T4*)(src + c0);
  const T4 wv = *(const T4*)(w + c0);
  float v[4], ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = (float)xv[i];
    ss = __builtin_fmaf(v[i], v[i], ss);
  }
  const float inv = rsqrtf(wave_sum(ss) / 256.f + eps);
  const int half = rd / 2, pos = t % L;
  T4 o;
  float nv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) nv[i] = round_through<bf16>(v[i] * inv * (1.f + (float)wv[i]));
  float pv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) pv[i] = __shfl_xor(nv[i], rd / 8);
  if (c0 < rd) {
    const T4 cs = *(const T4*)(cosb + (long long)pos * rd + c0), sn = *(const T4*)(sinb + (long long)pos * rd + c0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float rot = c0 < half ? -pv[i] : pv[i];
      o[i] = (bf16)round_through<bf16>(round_through<bf16>(nv[i] * (float)cs[i]) + round_through<bf16>(rot * (float)sn[i]));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (bf16)nv[i];
  }
  *(T4*)((isq ? qo : ko) + rr * 256 + c0) = o;
}

// The same over rows whose gate and up halves sit ld elements apart row to row (the two halves of
// one gate | up projection): out [rows, cols] contiguous; cols a multiple of 8.
template <typename T>
__global__ __launch_bounds__(256) void swiglu_rows_kernel(const T* __restrict__ g, const T* __restrict__ u,
                                                          long long ld, T* __restrict__ out, long long rows,
                                                          long long cols) {
  typedef __attribute__((ext_vector_type(8))) T V8;
  const long long i = ((long long)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i >= rows * cols) return;
  const long long r = i / cols, c = i - r * cols;
  const V8 gv = *(const V8*)(g + r * ld + c), uv = *(const V8*)(u + r * ld + c);
  V8 o;
#pragma unroll
  for (int k = 0; k < 8; ++k) o[k] = from_f32<T>(round_through<T>(silu_f32(to_f32(gv[k]))) * to_f32(uv[k]));
  *(V8*)(out + i) = o;
}

}  // namespace dllm

using namespace dllm;

template <typename T, typename TW>
static int launch_rmsnorm(const void* x, const void* r, void* so, const void* w, void* y, int rows, int dim, float eps,
                          int unit, bool vec, hipStream_t st) {
  const int nv = vec && dim % 512 == 0 && dim / 512 <= 16 ? dim / 512 : 0;
  if (nv > 1 && rows <= 256) {
    // few rows (a decoding step): one workgroup of up to 8 waves per row
    int nw = 8;
    while (nv % nw) --nw;
    const int nvw = nv / nw;
    switch (nvw) {
#define DLLM_RMS_ROW_CASE(N) \
  case N: rmsnorm_row_kernel<T, TW, N><<<dim3(rows), dim3(64 * nw), 0, st>>>((const T*)x, (const T*)r, (T*)so, (const TW*)w, (T*)y, dim, eps, unit); break;
      DLLM_RMS_ROW_CASE(1) DLLM_RMS_ROW_CASE(2) DLLM_RMS_ROW_CASE(3) DLLM_RMS_ROW_CASE(4) DLLM_RMS_ROW_CASE(5)
      DLLM_RMS_ROW_CASE(6) DLLM_RMS_ROW_CASE(7) DLLM_RMS_ROW_CASE(8)
#undef DLLM_RMS_ROW_CASE
      default: break;
    }
    if (nvw <= 8) {
      hipError_t e = hipGetLastError();
      return e == hipSuccess ? DLLM_OK : fail(DLLM_ELAUNCH, "rmsnorm launch: %s", hipGetErrorString(e));
    }
  }
  const dim3 grid((rows + 3) / 4), block(256);
  switch (nv) {
#define DLLM_RMS_CASE(N) \
  case N: rmsnorm_kernel<T, TW, N><<<grid, block, 0, st>>>((const T*)x, (const T*)r, (T*)so, (const TW*)w, (T*)y, rows, dim, eps, unit); break;
    DLLM_RMS_CASE(0) DLLM_RMS_CASE(1) DLLM_RMS_CASE(2) DLLM_RMS_CASE(3) DLLM_RMS_CASE(4) DLLM_RMS_CASE(5)
    DLLM_RMS_CASE(6) DLLM_RMS_CASE(7) DLLM_RMS_CASE(8) DLLM_RMS_CASE(9) DLLM_RMS_CASE(10) DLLM_RMS_CASE(11)
    DLLM_RMS_CASE(12) DLLM_RMS_CASE(13) DLLM_RMS_CASE(14) DLLM_RMS_CASE(15) DLLM_RMS_CASE(16)
#undef DLLM_RMS_CASE
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? DLLM_OK : fail(DLLM_ELAUNCH, "rmsnorm launch: %s", hipGetErrorString(e));
}

extern "C" int dllm_rmsnorm_fwd(const void* x, const void* residual, void* sum_out, const void* weight, void* y,
                                int rows, int dim, float eps, int dtype, int dtype_w, int unit_offset, void* stream) {
  if (!x || !weight || !y) return fail(DLLM_EINVAL, "rmsnorm: null pointer");
  if (rows < 0 || dim <= 0) return fail(DLLM_EINVAL, "rmsnorm: bad sizes rows=%d dim=%d", rows, dim);
  if (sum_out && !residual) return fail(DLLM_EINVAL, "rmsnorm: sum_out needs a residual");
  if (rows == 0) return DLLM_OK;
  const bool vec = ((uintptr_t)x | (uintptr_t)y | (uintptr_t)residual | (uintptr_t)sum_out | (uintptr_t)weight) % 16 == 0;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DT_BF16 && dtype_w == DT_BF16)
    return launch_rmsnorm<bf16, bf16>(x, residual, sum_out, weight, y, rows, dim, eps, unit_offset, vec, st);
  if (dtype == DT_BF16 && dtype_w == DT_F32)
    return launch_rmsnorm<bf16, float>(x, residual, sum_out, weight, y, rows, dim, eps, unit_offset, vec, st);
  if (dtype == DT_F32 && dtype_w == DT_F32)
    return launch_rmsnorm<float, float>(x, residual, sum_out, weight, y, rows, dim, eps, unit_offset, vec, st);
  return fail(DLLM_EUNSUPPORTED, "rmsnorm: dtype pair (%d, %d) not supported", dtype, dtype_w);
}

extern "C" int dllm_gated_rmsnorm_fwd(const void* x, const void* z, const void* weight, void* y, int rows, int dim,
                                      float eps, int dtype, int dtype_w, void* stream) {
  if (!x || !z || !weight || !y) return fail(DLLM_EINVAL, "gated rmsnorm: null pointer");
  if (rows < 0 || dim <= 0) return fail(DLLM_EINVAL, "gated rmsnorm: bad sizes rows=%d dim=%d", rows, dim);
  if (rows == 0) return DLLM_OK;
  hipStream_t st = (hipStream_t)stream;
  const bool vec = ((uintptr_t)x | (uintptr_t)z | (uintptr_t)weight | (uintptr_t)y) % 16 == 0;
  if (dtype == DT_BF16 && dtype_w == DT_BF16 && vec && (dim == 64 || dim == 128 || dim == 256 || dim == 512)) {
    const int rpb = 4 * (512 / dim);  // rows per workgroup: 4 waves of 64 / (dim / 8) rows
    const dim3 g((unsigned)((rows + rpb - 1) / rpb)), b(256);
    switch (dim) {
      case 64: gated_rmsnorm_vec_kernel<8><<<g, b, 0, st>>>((const bf16*)x, (const bf16*)z, (const bf16*)weight, (bf16*)y, rows, eps); break;
      case 128: gated_rmsnorm_vec_kernel<16><<<g, b, 0, st>>>((const bf16*)x, (const bf16*)z, (const bf16*)weight, (bf16*)y, rows, eps); break;
      case 256: gated_rmsnorm_vec_kernel<32><<<g, b, 0, st>>>((const bf16*)x, (const bf16*)z, (const bf16*)weight, (bf16*)y, rows, eps); break;
      default: gated_rmsnorm_vec_kernel<64><<<g, b, 0, st>>>((const bf16*)x, (const bf16*)z, (const bf16*)weight, (bf16*)y, rows, eps); break;
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? DLLM_OK : fail(DLLM_ELAUNCH, "gated rmsnorm launch: %s", hipGetErrorString(e));
  }
  const dim3 grid((rows + 3) / 4), block(256);
  if (dtype == DT_BF16 && dtype_w == DT_BF16)
    gated_rmsnorm_kernel<bf16, bf16><<<grid, block, 0, st>>>((const bf16*)x, (const bf16*)z, (const bf16*)weight,
                                                            (bf16*)y, rows, dim, eps);
  else if (dtype == DT_F32 && dtype_w == DT_F32)
    gated_rmsnorm_kernel<float, float><<<grid, block, 0, st>>>((const float*)x, (const float*)z,
                                                              (const float*)weight, (float*)y, rows, dim, eps);
  else
    return fail(DLLM_EUNSUPPORTED, "gated rmsnorm: dtype pair (%d, %d) not supported", dtype, dtype_w);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? DLLM_OK : fail(DLLM_ELAUNCH, "gated rmsnorm launch: %s", hipGetErrorString(e));
}

extern "C" int dllm_gdn_gates_fwd(const void* b, const void* a, const void* a_log, const void* dt_bias, float* beta,
                                  float* g, int64_t rows, int heads, int dtype, int dtype_param, void* stream) {
  if (!b || !a || !a_log || !dt_bias || !beta || !g) return fail(DLLM_EINVAL, "gdn gates: null pointer");
  if (rows <= 0 || heads <= 0) return fail(DLLM_EINVAL, "gdn gates: bad sizes rows=%lld heads=%d", (long long)rows, heads);
  const long long n = (long long)rows * heads;
  const long long nb = (n + 255) / 256;
  if (nb > 0x7fffffff) return fail(DLLM_EUNSUPPORTED, "gdn gates: too large");
  hipStream_t st = (hipStream_t)stream;
#define GATES(T, TP)                                                                                        \
  gdn_gates_kernel<T, TP><<<dim3((unsigned)nb), dim3(256), 0, st>>>((const T*)b, (const T*)a, (const TP*)a_log, \
                                                                   (const TP*)dt_bias, beta, g, n, heads)
  if (dtype == DT_BF16 && dtype_param == DT_F32) GATES(bf16, float);
  else if (dtype == DT_BF16 && dtype_param == DT_BF16) GATES(bf16, bf16);
  else if (dtype == DT_F32 && dtype_param == DT_F32) GATES(float, float);
  else if (dtype == DT_F32 && dtype_param == DT_BF16) GATES(float, bf16);
  else return fail(DLLM_EUNSUPPORTED, "gdn gates: dtype pair (%d, %d) not supported", dtype, dtype_param);
#undef GATES
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? DLLM_OK : fail(DLLM_ELAUNCH, "gdn gates launch: %s", hipGetErrorString(e));
}

extern "C" int dllm_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream) {
  if (!gate || !up || !out) return fail(DLLM_EINVAL, "swiglu: null pointer");
  if (n < 0) return fail(DLLM_EINVAL, "swiglu: bad size %lld", n);
  if (n == 0) return DLLM_OK;
  if (((uintptr_t)gate | (uintptr_t)up | (uintptr_t)out) % 16)
    return fail(DLLM_EINVAL, "swiglu: pointers must be 16-byte aligned");
  const long long nb = (n + 8 * 256 - 1) / (8 * 256);
  if (nb > 0x7fffffff) return fail(DLLM_EUNSUPPORTED, "swiglu: too large");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DT_BF16)
    swiglu_kernel<bf16><<<dim3((unsigned)nb), dim3(256), 0, st>>>((const bf16*)gate, (const bf16*)up, (bf16*)out, n);
  else if (dtype == DT_F32)
    swiglu_kernel<float><<<dim3((unsigned)nb), dim3(256), 0, st>>>((const float*)gate, (const float*)up, (float*)out, n);
  else
    return fail(DLLM_EUNSUPPORTED, "swiglu: dtype %d not supported", dtype);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? DLLM_OK : fail(DLLM_ELAUNCH, "swiglu launch: %s", hipGetErrorString(e));
}

extern "C" int dllm_swiglu_rows_fwd(const void* gate, const void* up, int64_t ld, void* out, int64_t rows,
                                    int64_t cols, int dtype, void* stream) {
  if (!gate || !up || !out) return fail(DLLM_EINVAL, "swiglu: null pointer");
  if (rows < 0 || cols < 0 || ld < cols) return fail(DLLM_EINVAL, "swiglu: bad sizes rows=%lld cols=%lld ld=%lld",
                                                      (long long)rows, (long long)cols, (long long)ld);
  if (rows == 0 || cols == 0) return DLLM_OK;
  if (cols % 8 || ld % 8 || ((uintptr_t)gate | (uintptr_t)up | (uintptr_t)out) % 16)
    return fail(DLLM_EINVAL, "swiglu: rows must be whole 16-byte vectors (cols, ld multiples of 8, aligned pointers)");
  const long long nb = (rows * cols + 8 * 256 - 1) / (8 * 256);
  if (nb > 0x7fffffff) return fail(DLLM_EUNSUPPORTED, "swiglu: too large");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DT_BF16)
    swiglu_rows_kernel<bf16><<<dim3((unsigned)nb), dim3(256), 0, st>>>((const bf16*)gate, (const bf16*)up, ld,
                                                                       (bf16*)out, rows, cols);
  else if (dtype == DT_F32)
    swiglu_rows_kernel<float><<<dim3((unsigned)nb), dim3(256), 0, st>>>((const float*)gate, (const float*)up, ld,
                                                                        (float*)out, rows, cols);
  else
    return fail(DLLM_EUNSUPPORTED, "swiglu: dtype %d not supported", dtype);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? DLLM_OK : fail(DLLM_ELAUNCH, "swiglu launch: %s", hipGetErrorString(e));
}

extern "C" int dllm_qk_norm_rope_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                                     const void* q_norm_w, const void* k_norm_w, const void* cos_table,
                                     const void* sin_table, void* q_out, void* k_out, int B, int S, int L, int Hq,
                                     int Hkv, int head_dim, int rotary_dim, float eps, int dtype, int dtype_w,
                                     void* stream) {
  // Hq == 0: the k rows alone (q, q_strides, q_norm_w and q_out may then be null)
  if ((Hq > 0 && (!q || !q_strides || !q_norm_w || !q_out)) || !k || !k_strides || !k_norm_w || !k_out)
    return fail(DLLM_EINVAL, "qk norm rope: null pointer");
  static const int64_t zero3[3] = {0, 0, 0};
  if (Hq == 0) q_strides = zero3;
  if (B <= 0 || S <= 0 || L <= 0 || Hq < 0 || Hkv <= 0 || head_dim <= 0 || head_dim > 256 || rotary_dim < 0 ||
      rotary_dim > head_dim || (rotary_dim & 1))
    return fail(DLLM_EINVAL, "qk norm rope: bad sizes B=%d S=%d L=%d Hq=%d Hkv=%d hd=%d rd=%d", B, S, L, Hq, Hkv,
                head_dim, rotary_dim);
  if (rotary_dim > 0 && (!cos_table || !sin_table)) return fail(DLLM_EINVAL, "qk norm rope: null rotary table");
  for (int i = 1; i < 3; ++i)
    if (q_strides[i] > 0x7fffffff || k_strides[i] > 0x7fffffff)
      return fail(DLLM_EUNSUPPORTED, "qk norm rope: token/head strides exceed 32 bits");
  const long long rows = (long long)B * S * (Hq + Hkv);
  const long long nb = (rows + 3) / 4;
  if (nb > 0x7fffffff) return fail(DLLM_EUNSUPPORTED, "qk norm rope: too large");
  hipStream_t st = (hipStream_t)stream;
  const int rd8 = rotary_dim / 8;
  const bool rd_ok = rotary_dim > 0 && rotary_dim % 8 == 0 && (rd8 & (rd8 - 1)) == 0;
  const bool al8 = ((uintptr_t)q | (uintptr_t)k | (uintptr_t)q_norm_w | (uintptr_t)k_norm_w | (uintptr_t)cos_table |
                    (uintptr_t)sin_table | (uintptr_t)q_out | (uintptr_t)k_out) % 8 == 0;
  bool st4 = true;
  for (int i = 0; i < 3; ++i) st4 = st4 && q_strides[i] % 4 == 0 && k_strides[i] % 4 == 0;
  if (dtype == DT_BF16 && dtype_w == DT_BF16 && head_dim == 256 && rd_ok && al8 && st4) {
    qk_norm_rope256_kernel<<<dim3((unsigned)nb), dim3(256), 0, st>>>(
        (const bf16*)q, q_strides[0], (int)q_strides[1], (int)q_strides[2], (const bf16*)k, k_strides[0],
        (int)k_strides[1], (int)k_strides[2], (const bf16*)q_norm_w, (const bf16*)k_norm_w, (const bf16*)cos_table,
        (const bf16*)sin_table, (bf16*)q_out, (bf16*)k_out, B, S, L, Hq, Hkv, rotary_dim, eps);
  } else if (dtype == DT_BF16 && dtype_w == DT_BF16)
    qk_norm_rope_kernel<bf16, bf16><<<dim3((unsigned)nb), dim3(256), 0, st>>>(
        (const bf16*)q, q_strides[0], (int)q_strides[1], (int)q_strides[2], (const bf16*)k, k_strides[0],
        (int)k_strides[1], (int)k_strides[2], (const bf16*)q_norm_w, (const bf16*)k_norm_w, (const bf16*)cos_table,
        (const bf16*)sin_table, (bf16*)q_out, (bf16*)k_out, B, S, L, Hq, Hkv, head_dim, rotary_dim, eps);
  else if (dtype == DT_BF16 && dtype_w == DT_F32)  // norm weights kept in fp32 beside bf16 activations
    qk_norm_rope_kernel<bf16, float><<<dim3((unsigned)nb), dim3(256), 0, st>>>(
        (const bf16*)q, q_strides[0], (int)q_strides[1], (int)q_strides[2], (const bf16*)k, k_strides[0],
        (int)k_strides[1], (int)k_strides[2], (const float*)q_norm_w, (const float*)k_norm_w, (const bf16*)cos_table,
        (const bf16*)sin_table, (bf16*)q_out, (bf16*)k_out, B, S, L, Hq, Hkv, head_dim, rotary_dim, eps);
  else if (dtype == DT_F32 && dtype_w == DT_F32)
    qk_norm_rope_kernel<float, float><<<dim3((unsigned)nb), dim3(256), 0, st>>>(
        (const float*)q, q_strides[0], (int)q_strides[1], (int)q_strides[2], (const float*)k, k_strides[0],
        (int)k_strides[1], (int)k_strides[2], (const float*)q_norm_w, (const float*)k_norm_w, (const float*)cos_table,
        (const float*)sin_table, (float*)q_out, (float*)k_out, B, S, L, Hq, Hkv, head_dim, rotary_dim, eps);
  else
    return fail(DLLM_EUNSUPPORTED, "qk norm rope: dtype pair (%d, %d) not supported", dtype, dtype_w);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? DLLM_OK : fail(DLLM_ELAUNCH, "qk norm rope launch: %s", hipGetErrorString(e));
}
