// Shared device/host helpers for the gfx950 (CDNA4) kernels of the block-diffusion forward.
//
// MFMA fragment convention used by every kernel in this library
// ---------------------------------------------------------------
// All matrix products are built from 32x32 output tiles (v_mfma_f32_32x32x16_bf16 for bf16
// operands, v_mfma_f32_32x32x2f32 for fp32 operands), accumulated in fp32.
//
// The 32x32 fp32 accumulator (f32x16) of lane l holds column j = l % 32 and, for value index
// v = 0..15, row  rho(v, h) = 8*(v/4) + 4*h + (v%4)  with h = l / 32.
//
// Products contract over K in units of 32. For a 32-wide K slice, every operand is supplied by
// lane (row-or-column = l % 32, half h = l / 32) as 16 values in the SAME rho order:
// value v of the fragment carries k = rho(v, h). For bf16 MFMA, instruction u (0,1) consumes
// values 8u..8u+7; for fp32 MFMA, instruction s (0..15) consumes value s. Since A and B use the
// same (h, slot) -> k assignment, the hardware contracts matching k indices whatever its own
// k numbering is, and an accumulator can be fed back as a B operand without any data movement:
// its rows are already in rho order.
//
// Reading a rho-ordered fragment from a [row][k] array with k contiguous is four runs of four
// consecutive elements at k = 8m + 4h (m = 0..3): two 8-byte LDS reads per MFMA in bf16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dllm_hip.h"  // every entry point's definition is checked against its declaration

namespace dllm {

typedef __bf16 bf16;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

// dtype codes of the C ABI
enum { DT_F32 = 0, DT_BF16 = 1 };

__device__ __forceinline__ int rho(int v, int h) { return ((v >> 2) << 3) + (h << 2) + (v & 3); }

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }

// Round an fp32 value through type T (identity for float).
template <typename T> __device__ __forceinline__ float round_through(float x) { return to_f32(from_f32<T>(x)); }

// Sum over the 64 lanes of a wave, returned to every lane (butterfly: strides 32, 16, .., 1).
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// SiLU x * sigmoid(x) from the hardware base-2 exponential and reciprocal (each within 1 ulp):
// within a few fp32 ulp of x / (1 + e^-x); large negative x gives -0 where the exact value underflows.
__device__ __forceinline__ float silu_f32(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// Fragment: 16 rho-ordered operand values for one 32-wide K slice.
template <bool BF16> struct Frag;
template <> struct Frag<true> { bf16x8 lo, hi; };     // values 0..7 and 8..15
template <> struct Frag<false> { float v[16]; };

// Fragment from an accumulator tile (values already in rho order), optionally row-scaled.
__device__ __forceinline__ void acc_to_frag(const f32x16& a, Frag<true>& f) {
#pragma unroll
  for (int i = 0; i < 8; ++i) { f.lo[i] = (bf16)a[i]; f.hi[i] = (bf16)a[i + 8]; }
}
__device__ __forceinline__ void acc_to_frag(const f32x16& a, Frag<false>& f) {
#pragma unroll
  for (int i = 0; i < 16; ++i) f.v[i] = a[i];
}

// Fragment from LDS: base points at element k = 0 of this lane's row (row stride irrelevant).
__device__ __forceinline__ void lds_frag(const bf16* base, int h, Frag<true>& f) {
  const bf16x4 r0 = *(const bf16x4*)(base + 4 * h);
  const bf16x4 r1 = *(const bf16x4*)(base + 8 + 4 * h);
  const bf16x4 r2 = *(const bf16x4*)(base + 16 + 4 * h);
  const bf16x4 r3 = *(const bf16x4*)(base + 24 + 4 * h);
  f.lo = __builtin_shufflevector(r0, r1, 0, 1, 2, 3, 4, 5, 6, 7);
  f.hi = __builtin_shufflevector(r2, r3, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ void lds_frag(const float* base, int h, Frag<false>& f) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const f32x4 r = *(const f32x4*)(base + 8 * m + 4 * h);
    f.v[4 * m + 0] = r[0]; f.v[4 * m + 1] = r[1]; f.v[4 * m + 2] = r[2]; f.v[4 * m + 3] = r[3];
  }
}

// Fragment of the TRANSPOSED access to a row-major bf16 buffer: lane (l32, h) gets column
// col0 + l32 at rows (k) 8m + 4h + e, e = 0..3 (rho order), where base points at (row 0, col0).
// Uses the gfx950 LDS transpose read: in each group of 16 lanes, source lane s supplies the
// address of 4 consecutive columns (4 (s & 3) onwards) of row (s >> 2), and result lane i receives
// column i of those 4 rows. Row stride and col0 must keep every address 8-byte aligned.
__device__ __forceinline__ void lds_frag_tr(const bf16* base, int row_stride, int lane, Frag<true>& f) {
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  const int s = lane & 15;
  const bf16* p = base + (4 * (lane >> 5) + (s >> 2)) * row_stride + 16 * ((lane >> 4) & 1) + 4 * (s & 3);
  bf16x4 r[4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
    r[m] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p + 8 * m * row_stride));
  f.lo = __builtin_shufflevector(r[0], r[1], 0, 1, 2, 3, 4, 5, 6, 7);
  f.hi = __builtin_shufflevector(r[2], r[3], 0, 1, 2, 3, 4, 5, 6, 7);
}

// acc += A_frag * B_frag over one 32-wide K slice.
__device__ __forceinline__ void mma32(f32x16& acc, const Frag<true>& a, const Frag<true>& b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.lo, b.lo, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.hi, b.hi, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma32(f32x16& acc, const Frag<false>& a, const Frag<false>& b) {
#pragma unroll
  for (int s = 0; s < 16; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.v[s], b.v[s], acc, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Direct global -> LDS load of 16 bytes per lane: lane i's 16 bytes land at lds_base + 16 i
// (lds_base wave-uniform). Emitted as inline assembly: the compiler cannot tell a kernel's LDS
// stage buffers apart, so for its own load-to-LDS builtin it waits for every such load in flight
// before each later LDS read and at every barrier, which serialises a prefetch ring. Callers wait
// for these loads with explicit vmcnt counts.
__device__ __forceinline__ void dma_load16(const void* src, const void* lds_base) {
  typedef const __attribute__((address_space(3))) void* lds_cptr;
  const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(lds_cptr)lds_base);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}
// The same for data read once per launch and never again soon (streamed weights): non-temporal
// at device scope, so the lines do not displace reused data in the L2 and the last-level cache.
__device__ __forceinline__ void dma_load16_stream(const void* src, const void* lds_base) {
  typedef const __attribute__((address_space(3))) void* lds_cptr;
  const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(lds_cptr)lds_base);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt sc1" ::"v"(src), "s"(m0) : "memory", "m0");
}

// Ordering point for LDS traffic between lanes of ONE wavefront (no s_barrier): LDS operations of
// a wave complete in issue order, so only compiler reordering has to be prevented.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Fork index functions (state fork of the block-diffusion forward), shared by the conv kernel,
// the layout kernel and the host: row of (sequence b, block k); flat clean-state index a row
// starts from (-1 = zero state); clean position feeding conv-prefix slot j (-1 = zero padding).
__host__ __device__ __forceinline__ int fork_row(int b, int k, int nb) { return b * nb + k; }
__host__ __device__ __forceinline__ int fork_state_src(int b, int k, int nb) { return k == 0 ? -1 : b * nb + k - 1; }
__host__ __device__ __forceinline__ int fork_prefix_pos(int k, int j, int block, int width) {
  const int p = k * block - (width - 1) + j;
  return p >= 0 ? p : -1;
}

}  // namespace dllm

// ---- host-side error reporting shared by the C ABI ----
namespace dllm {
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
}  // namespace dllm

// status codes of the C ABI (negative = error)
#define DLLM_OK 0
#define DLLM_EINVAL (-1)
#define DLLM_EUNSUPPORTED (-2)
#define DLLM_ELAUNCH (-3)
