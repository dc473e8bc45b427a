// Block-diffusion attention with the complementary [2L, 2L] mask (gfx950 / CDNA4).
//
// Sequence = cat([x_t, x_0]) of length 2L, blocks of C tokens, positions kept per half. Query i may
// see key j iff (with qb, kb the blocks inside each half):
//   x_t -> x_t : kb == qb   (kb <= qb under the "mask-leak" fault)
//   x_t -> x_0 : kb <  qb
//   x_0 -> x_0 : kb <= qb
//   x_0 -> x_t : never
// The mask is never materialised: a workgroup takes four 32-query tiles of one half and one query
// head; it walks only the 32-key tiles that the union of its rows can see, and each wave skips the
// tiles its own rows cannot see. With C = 32 every (32-query, 32-key) tile is entirely visible or
// entirely hidden, so no element masks are evaluated; other block sizes and ragged lengths mask
// elements on the partial tiles only.
//
// Per wave and key tile: S^T = K Q^T on MFMA (rows = keys, lane = query), online softmax in fp32
// with exp2, P rounded to the input dtype, then O^T += V^T P^T on MFMA: the accumulator layout of
// S^T is directly the B-operand layout of P^T, and each lane owns one query column of O^T, so the
// softmax rescale is a per-lane scalar (applied lazily, only when a running maximum grows by more
// than 2^8). K and V tiles are staged row-major in a double-buffered LDS ring (bf16 V^T operands
// come from gfx950 LDS transpose reads), the next tile's global loads travelling during the current
// compute.
// GQA: query head h reads KV head h / (Hq / Hkv), no repeat_kv copy.
//
// Block-causal mode (template flag BC): one sequence of N keys at absolute positions 0..N-1 (a
// cached clean prefix plus the current segment) and M query rows at absolute positions q0..q0+M-1;
// query i sees key j iff j / C <= (q0 + i) / C. It is the x_0 -> x_0 rule above with the query rows
// offset, so the kernels run it as half 1 with its own row counts: a decode step (M = C, q0 = N - C,
// every key visible) and the prefill of a prompt (q0 = 0, M = N) are both this mode.
#include <type_traits>

#include "common.h"

namespace dllm {

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;  // [B, 2L, Hq, d] contiguous
  long long q_sb, k_sb, v_sb;
  int q_st, q_sh, k_st, k_sh, v_st, v_sh;
  int B, L, Hq, Hkv, d, C;
  int leak;
  int M, N, q0;       // block-causal mode: query rows, key rows, absolute position of query row 0
  int ksplit;         // block-causal mode, direct-load kernel: key tiles split over grid.y
  float* opart;       // ksplit > 1: unnormalised O [ksplit][B][M][Hq][d] fp32
  float* mlpart;      // ksplit > 1: running max and sum [ksplit][B][M][Hq][2] fp32
  float scale_log2e;  // softmax scale * log2(e)
  int vec;            // 16-byte vector loads of q/k/v rows allowed
  // gated attention layer, fused (direct-load kernel, complementary-mask mode only):
  // q_norm_w non-null: q is the raw q_proj output; each query row is RMSNorm(1 + w)-normalised and
  // its first `rd` dims rotated (rotate_half, position = row index within its half) as it is
  // loaded, with the rounding of the separate q/k norm + RoPE kernel
  const void* q_norm_w;
  int q_norm_f32;  // the weight is fp32 (else bf16)
  float q_eps;
  const void* cosb;  // [L, rd] rotary tables in the activation dtype
  const void* sinb;
  int rd;
  // gate non-null: out = attention * sigmoid(gate), gate [B, 2L, Hq, d] (block-causal mode:
  // [B, M, Hq, d]) with these strides
  const void* gate;
  long long g_sb;
  int g_st, g_sh;
};

// Work unit of dispatch slot bid among n. The dispatcher hands slot bid to XCD bid % 8, in order of
// bid / 8 within an XCD. Units are numbered longest first, in chunks of `chunk` consecutive units
// that read the same K/V head; chunk c runs on XCD c % 8, so that every XCD receives an equal share
// of each length class (a contiguous range per XCD would give one XCD all the longest units) and a
// K/V head's tiles are shared through that XCD's L2. Slots past the last whole row of eight chunks
// map to themselves. A bijection of [0, n).
__device__ __forceinline__ int attn_unit(int bid, int n, int chunk) {
  const int full = n / (8 * chunk) * (8 * chunk);
  if (bid >= full) return bid;
  const int x = bid & 7, i = bid >> 3;
  return ((i / chunk) * 8 + x) * chunk + i % chunk;
}

// visibility of key block kb of half kh from query block qb of half qh (0 = x_t, 1 = x_0)
__device__ __forceinline__ bool visible(int qh, int qb, int kh, int kb, int leak) {
  if (qh == 0) return kh == 0 ? (leak ? kb <= qb : kb == qb) : (kb < qb);
  return kh == 1 && kb <= qb;
}

// any / all of the query-block range [q0, q1] x key-block range [k0, k1] visible
__device__ __forceinline__ void classify(int qh, int q0, int q1, int kh, int k0, int k1, int leak, bool& any,
                                         bool& all) {
  if (qh == 1 && kh == 0) { any = all = false; return; }
  if (qh == 0 && kh == 0 && !leak) {
    any = (k0 <= q1) && (q0 <= k1);
    all = (q0 == q1) && (k0 == k1) && (k0 == q0);
    return;
  }
  if (qh == 0 && kh == 1) {  // kb < qb
    any = k0 < q1;
    all = k1 < q0;
    return;
  }
  any = k0 <= q1;  // kb <= qb
  all = k1 <= q0;
}

template <int D, bool BF16>
struct AttnSmem {
  using OpT = typename std::conditional<BF16, bf16, float>::type;
  static constexpr int KROW = D + (BF16 ? 8 : 4);  // K tile [32][D]
  // bf16: V tile row-major [32][D] (V^T operands come from LDS transpose reads); fp32: V^T [D][32]
  static constexpr int VROW = BF16 ? D + 8 : 36;
  static constexpr int K_BYTES = 32 * KROW * (int)sizeof(OpT);
  static constexpr int V_BYTES = (BF16 ? 32 : D) * VROW * (int)sizeof(OpT);
  static constexpr int STAGE = K_BYTES + V_BYTES;
  static constexpr int TOTAL = 2 * STAGE;
};

template <int D, bool BF16, bool BC>
__global__ __launch_bounds__(256) void bd_attn_kernel(AttnArgs a) {
  using SM = AttnSmem<D, BF16>;
  using OpT = typename SM::OpT;
  using F = Frag<BF16>;
  constexpr int DT = D / 32;
  constexpr int KROW = SM::KROW, VROW = SM::VROW;
  constexpr int EPV = 16 / (int)sizeof(OpT);  // elements per 16-byte vector
  constexpr int CPR = D / EPV;                // 16-byte chunks per row
  constexpr int CPT = CPR >= 8 ? CPR / 8 : 1;  // chunks per thread per tile (K or V); 8 threads per row
  using V16 = typename std::conditional<BF16, bf16x8, f32x4>::type;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SM::TOTAL];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int L = a.L, C = a.C;
  const int Lq = BC ? a.M : L;     // query rows per half
  const int Lk = BC ? a.N : L;     // key rows per half
  const int qa = BC ? a.q0 : 0;    // absolute position of query row 0
  const int ntq = (Lq + 31) >> 5;  // 32-row tiles per half
  const int ng = (ntq + 3) >> 2;  // groups of four tiles per half
  const int rep = a.Hq / a.Hkv;

  // work unit: longest first (tile group descending), then half, batch, KV head, query head in group
  constexpr int NH = BC ? 1 : 2;  // query halves
  const int lin = attn_unit(blockIdx.x, gridDim.x, NH * rep);
  const int per_g = NH * a.B * a.Hkv * rep;
  const int g = ng - 1 - lin / per_g;
  int rem = lin % per_g;
  const int qh = BC ? 1 : rem % 2;  // alternate halves so equal-work units sit together
  rem /= NH;
  const int hr = rem % rep;
  rem /= rep;
  const int hkv = rem % a.Hkv;
  const int b = rem / a.Hkv;
  const int hq = hkv * rep + hr;

  // this wave's query rows [r0, r1) inside half qh; the workgroup's rows [g0, g1)
  const int g0 = g * 128, g1 = min(Lq, g0 + 128);
  const int r0 = g0 + wave * 32, r1 = min(Lq, r0 + 32);
  const bool wave_live = r0 < Lq;
  const int qb0 = (qa + r0) / C, qb1 = (qa + max(r0, r1 - 1)) / C;
  const int gqb0 = (qa + g0) / C, gqb1 = (qa + g1 - 1) / C;

  // key ranges of the workgroup, per half: [lo, hi) in tokens
  int lo0, hi0, lo1, hi1;  // half 0 (x_t) and half 1 (x_0)
  if (qh == 1) {
    lo0 = hi0 = 0;
    lo1 = 0;
    hi1 = min(Lk, (gqb1 + 1) * C);
  } else {
    lo0 = a.leak ? 0 : gqb0 * C;
    hi0 = min(L, (gqb1 + 1) * C);
    lo1 = 0;
    hi1 = min(L, gqb1 * C);
  }
  const int t0lo = lo0 >> 5, t0hi = (hi0 + 31) >> 5;  // x_t key tiles
  const int t1lo = lo1 >> 5, t1hi = (hi1 + 31) >> 5;  // x_0 key tiles
  const int n0 = hi0 > lo0 ? t0hi - t0lo : 0;
  const int n1 = hi1 > lo1 ? t1hi - t1lo : 0;
  const int ntiles = n0 + n1;  // x_0 tiles first, then x_t tiles
  auto tile_pos = [&](int n, int& kh, int& j0) {
    if (n < n1) { kh = 1; j0 = (t1lo + n) * 32; }
    else { kh = 0; j0 = (t0lo + n - n1) * 32; }
  };

  const OpT* const qbase = (const OpT*)a.q + b * a.q_sb + (long long)hq * a.q_sh;
  const OpT* const kbase = (const OpT*)a.k + b * a.k_sb + (long long)hkv * a.k_sh;
  const OpT* const vbase = (const OpT*)a.v + b * a.v_sb + (long long)hkv * a.v_sh;

  // Q^T fragments for this wave's 32 queries (lane = query, d in rho order), kept in registers
  F qf[DT];
  {
    const int row = min(r0 + l32, Lq - 1);  // rows past the end load a valid row and are never stored
    const OpT* qp = qbase + (long long)((BC ? 0 : qh * L) + row) * a.q_st;
#pragma unroll
    for (int s = 0; s < DT; ++s) {
      if constexpr (BF16) {
        bf16x4 r[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int d0 = 32 * s + 8 * m + 4 * h;
#pragma unroll
          for (int e = 0; e < 4; ++e) r[m][e] = (d0 + e < a.d) ? qp[d0 + e] : from_f32<OpT>(0.f);
        }
        qf[s].lo = __builtin_shufflevector(r[0], r[1], 0, 1, 2, 3, 4, 5, 6, 7);
        qf[s].hi = __builtin_shufflevector(r[2], r[3], 0, 1, 2, 3, 4, 5, 6, 7);
      } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int dd = 32 * s + rho(v, h);
          qf[s].v[v] = dd < a.d ? qp[dd] : 0.f;
        }
      }
    }
  }

  // key/value tile staging: thread -> (key row kr, chunks {kc + 8q}) of K and of V
  const int kr = tid >> 3, kc = tid & 7;
  V16 rk[CPT], rv[CPT];
  const V16 vz = {};
  auto load_tile = [&](int n) {
    int kh, j0;
    tile_pos(n, kh, j0);
    const int key = j0 + kr;
    const bool ok = key < Lk;
    const int krow = (BC ? 0 : kh * L) + (ok ? key : 0);
    const OpT* kp = kbase + (long long)krow * a.k_st;
    const OpT* vp = vbase + (long long)krow * a.v_st;
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      if (kc + 8 * q >= CPR) continue;
      const int e0 = (kc + 8 * q) * EPV;
      if (a.vec) {
        rk[q] = *(const V16*)(kp + e0);
        rv[q] = *(const V16*)(vp + e0);
      } else {
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
          rk[q][e] = (e0 + e < a.d) ? kp[e0 + e] : from_f32<OpT>(0.f);
          rv[q][e] = (e0 + e < a.d) ? vp[e0 + e] : from_f32<OpT>(0.f);
        }
      }
    }
  };
  auto store_tile = [&](int n, int stage) {
    int kh, j0;
    tile_pos(n, kh, j0);
    const bool ok = j0 + kr < Lk;
    OpT* Ks = (OpT*)(smem + stage * SM::STAGE);
    OpT* Vs = (OpT*)(smem + stage * SM::STAGE + SM::K_BYTES);
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      if (kc + 8 * q >= CPR) continue;
      const int e0 = (kc + 8 * q) * EPV;
      const V16 kx = ok ? rk[q] : vz;
      const V16 vx = ok ? rv[q] : vz;
      *(V16*)(Ks + kr * KROW + e0) = kx;
      if constexpr (BF16) {
        *(V16*)(Vs + kr * VROW + e0) = vx;
      } else {
#pragma unroll
        for (int e = 0; e < EPV; ++e) Vs[(e0 + e) * VROW + kr] = vx[e];
      }
    }
  };

  f32x16 O[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) O[t] = zero16();
  float mrow = -1e30f, lrow = 0.f;  // running max (log2 units) and sum of this lane's query

  if (ntiles > 0) {
    load_tile(0);
    store_tile(0, 0);
  }
  __syncthreads();
  for (int n = 0; n < ntiles; ++n) {
    if (n + 1 < ntiles) load_tile(n + 1);
    int kh, j0;
    tile_pos(n, kh, j0);
    const int kb0 = j0 / C, kb1 = (min(Lk, j0 + 32) - 1) / C;
    bool any = false, all = false;
    if (wave_live) classify(qh, qb0, qb1, kh, kb0, kb1, a.leak, any, all);
    const bool ragged = (j0 + 32 > Lk) || (r1 - r0 < 32);
    if (any) {
      const OpT* Ks = (const OpT*)(smem + (n & 1) * SM::STAGE);
      const OpT* Vs = (const OpT*)(smem + (n & 1) * SM::STAGE + SM::K_BYTES);
      // S^T = K Q^T : rows = keys (rho order), lane = query
      f32x16 st = zero16();
      constexpr int KB = DT >= 4 ? 4 : DT;
#pragma unroll
      for (int s0 = 0; s0 < DT; s0 += KB) {
        F kf[KB];
#pragma unroll
        for (int s = 0; s < KB; ++s) lds_frag(Ks + l32 * KROW + 32 * (s0 + s), h, kf[s]);
#pragma unroll
        for (int s = 0; s < KB; ++s) mma32(st, kf[s], qf[s0 + s]);
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) st[v] *= a.scale_log2e;
      if (!all || ragged) {
        const int qi = r0 + l32;
        const int qbl = (qa + qi) / C;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int kj = j0 + rho(v, h);
          const bool okk = kj < Lk && qi < Lq && visible(qh, qbl, kh, kj / C, a.leak);
          st[v] = okk ? st[v] : -INFINITY;
        }
      }
      float mx = st[0];
#pragma unroll
      for (int v = 1; v < 16; ++v) mx = fmaxf(mx, st[v]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // Lazy rescale: the reference maximum moves only when some lane's tile maximum exceeds it by
      // more than RESCALE_LOG2 (then O and l are rescaled, wave-uniformly); otherwise the
      // unnormalised probabilities stay below 2^RESCALE_LOG2 and O, l keep accumulating against the
      // same reference. O / l is unchanged; most tiles skip the O rescale entirely.
      constexpr float RESCALE_LOG2 = 8.f;
      if (__builtin_amdgcn_ballot_w64(mx > mrow + RESCALE_LOG2) != 0) {
        const float mnew = fmaxf(mrow, mx);
        const float alpha = __builtin_amdgcn_exp2f(mrow - mnew);
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int v = 0; v < 16; ++v) O[t][v] *= alpha;
        lrow *= alpha;
        mrow = mnew;
      }
      float ps = 0.f;
      f32x16 p;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        p[v] = __builtin_amdgcn_exp2f(st[v] - mrow);
        ps += p[v];
      }
      ps += __shfl_xor(ps, 32);
      lrow += ps;
      F pf;
      acc_to_frag(p, pf);
      // O^T += V^T P^T
      constexpr int VB = DT >= 4 ? 4 : DT;
#pragma unroll
      for (int t0 = 0; t0 < DT; t0 += VB) {
        F vf[VB];
#pragma unroll
        for (int t = 0; t < VB; ++t) {
          if constexpr (BF16) {
            lds_frag_tr(Vs + 32 * (t0 + t), VROW, lane, vf[t]);
          } else {
            lds_frag(Vs + (32 * (t0 + t) + l32) * VROW, h, vf[t]);
          }
        }
#pragma unroll
        for (int t = 0; t < VB; ++t) mma32(O[t0 + t], vf[t], pf);
      }
    }
    if (n + 1 < ntiles) store_tile(n + 1, (n + 1) & 1);
    __syncthreads();
  }

  // O = (O^T)^T / l : lane = query row, four runs of four consecutive d per 32-slice
  const int qi = r0 + l32;
  if (wave_live && qi < Lq) {
    const float inv = 1.f / lrow;
    const long long orow = BC ? (long long)b * Lq + qi : (long long)b * 2 * L + qh * L + qi;
    OpT* op = (OpT*)a.out + (orow * a.Hq + hq) * a.d;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int d0 = 32 * t + 8 * m + 4 * h;
        if constexpr (BF16) {
          if (d0 + 4 <= a.d && (a.d & 3) == 0) {
            bf16x4 o4;
#pragma unroll
            for (int e = 0; e < 4; ++e) o4[e] = (bf16)(O[t][4 * m + e] * inv);
            *(bf16x4*)(op + d0) = o4;
            continue;
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (d0 + e < a.d) op[d0 + e] = from_f32<OpT>(O[t][4 * m + e] * inv);
      }
  }
}

template <int D, bool BF16, bool BC>
static int launch_attn(const AttnArgs& a, hipStream_t st) {
  const int ntq = ((BC ? a.M : a.L) + 31) / 32;
  const int ng = (ntq + 3) / 4;
  const long long nblk = (long long)ng * (BC ? 1 : 2) * a.B * a.Hq;
  if (nblk > 0x7fffffff) return fail(DLLM_EUNSUPPORTED, "attention: grid too large");
  bd_attn_kernel<D, BF16, BC><<<dim3((unsigned)nblk), dim3(256), 0, st>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "attention launch: %s", hipGetErrorString(e));
  return DLLM_OK;
}

// Chunk swizzle of a tile row: logical 16-byte chunk c of row r sits at physical chunk c ^ swz_key(r).
// LDS has 64 banks of 4 bytes; a 16-byte read is served 16 lanes per pass and an 8-byte read 32
// lanes per pass. The K fragment reads take one chunk of 16 consecutive rows per pass, so the key
// must be a bijection of the row's low bits; the V^T transpose reads take four chunks of each of
// four consecutive rows per pass, so the key must also put the row's lowest two bits above the
// chunk's lowest two. Swapping the row's two 2-bit fields does both for D = 128 and 256 (measured
// 4% and 8% faster than keying by the row alone). D = 64 keeps the plain row key, which measured
// faster there.
template <int D>
__device__ __forceinline__ int swz_key(int row) {
  constexpr int CH = D / 8;
  if constexpr (CH >= 16) return ((row & 3) << 2) | ((row >> 2) & 3);
  else return row & (CH - 1);
}

template <int D>
__device__ __forceinline__ int swz_off(int row, int col) {  // byte offset of (row, col) in a swizzled tile
  return row * (2 * D) + (((col >> 3) ^ swz_key<D>(row)) << 4) + ((col & 7) << 1);
}

// s_waitcnt with vmcnt(N) and the other counters unconstrained (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// ---------------------------------------------------------------------------------------------
// bf16, d == D in {64, 128, 256}: eight waves, a pair per 32-query tile, split by role.
// Waves 0..3 (S waves) hold Q^T of query tile u = wave and form S^T = K Q^T (lane = query), the mask
// and the online softmax; they hand P (the B-operand fragment of P^T, lane-major) and the rescale
// factor of each query to their partner through an LDS ring of two slots. Waves 4..7 (O waves)
// hold O^T of the same query tile over the whole d and, one key tile behind, apply the rescale and
// accumulate O^T += V^T P^T. No product is formed twice, an S wave holds no O and an O wave no Q,
// and each SIMD runs one wave of each kind. (A split of the pair by halves of d instead forms S in
// both waves: measured 1.25x the time at d = 256.) The hand-off needs no extra synchronisation:
// slot n % 2 is written in the phase of tile n and read in the phase of tile n + 1, across the one
// barrier per tile. The S waves are pipelined one tile ahead (the schedule is stated in the kernel).
// K and V tiles travel global -> LDS by direct loads, no registers: each wave instruction moves
// 1 KB = 64 lanes x 16 bytes; rows are dense with their 16-byte chunks XOR-swizzled (swz_key) so
// that the K fragment reads and the V^T transpose reads are free of bank conflicts. K and V have
// rings of their own, since a tile's K is read two phases before its V.
// ---------------------------------------------------------------------------------------------
// Max / sum of lane l's value and lane l ^ 32's (the two rows of an MFMA accumulator column),
// exchanged by the gfx950 lane swap between the wave halves instead of through LDS. The sum's
// operands are those of x + shfl_xor(x, 32), so both give the same bits.
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// RMSNorm(1 + w) and rotate_half RoPE of one query row held as the direct-load kernel's Q^T
// fragments (lane (row, h): slice s holds d = 32 s + 8 h + (0..7) in lo and 32 s + 16 + 8 h +
// (0..7) in hi, the other half of the row in lane ^ 32). The rounding follows the separate q/k
// norm + RoPE kernel (qk_norm_rope256_kernel): n = bf16((x / rms) (1 + w)), and in the first rd
// dims bf16(bf16(n cos) + bf16(+-partner sin)). The rotation pairs d with d + rd / 2, which with
// rd / 2 a multiple of 32 is the same position of slice s + rd / 64: in the same lane.
// rotate_half over slice pairs (s, s + NH), s < NH: d pairs with d + 32 NH (rotary_dim = 64 NH)
template <int D, int NH>
__device__ __forceinline__ void rope_pairs(Frag<true> (&qf)[D / 32], const bf16* cs, const bf16* sn, int h) {
#pragma unroll
  for (int s = 0; s < NH; ++s)
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      const int d1 = 32 * s + 16 * part + 8 * h, d2 = d1 + 32 * NH;
      const bf16x8 c1 = *(const bf16x8*)(cs + d1), s1 = *(const bf16x8*)(sn + d1);
      const bf16x8 c2 = *(const bf16x8*)(cs + d2), s2 = *(const bf16x8*)(sn + d2);
      bf16x8& x1 = part ? qf[s].hi : qf[s].lo;
      bf16x8& x2 = part ? qf[s + NH].hi : qf[s + NH].lo;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float a1 = (float)x1[i], a2 = (float)x2[i];
        const float o1 = (float)(bf16)((float)(bf16)(a1 * (float)c1[i]) + (float)(bf16)(-a2 * (float)s1[i]));
        const float o2 = (float)(bf16)((float)(bf16)(a2 * (float)c2[i]) + (float)(bf16)(a1 * (float)s2[i]));
        x1[i] = (bf16)o1;
        x2[i] = (bf16)o2;
      }
    }
}

template <int D>
__device__ __forceinline__ void q_norm_rope(Frag<true> (&qf)[D / 32], const AttnArgs& a, int pos, int h) {
  constexpr int DT = D / 32;
  // sum of squares from the bf16 pairs (paired dot products: no unpacked copy of the row is held)
  float ss = 0.f;
#pragma unroll
  for (int s = 0; s < DT; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bf16x2 lo = {qf[s].lo[2 * i], qf[s].lo[2 * i + 1]};
      const bf16x2 hi = {qf[s].hi[2 * i], qf[s].hi[2 * i + 1]};
      ss = __builtin_amdgcn_fdot2_f32_bf16(lo, lo, ss, false);
      ss = __builtin_amdgcn_fdot2_f32_bf16(hi, hi, ss, false);
    }
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
  const float inv = rsqrtf((__uint_as_float(r[0]) + __uint_as_float(r[1])) / (float)D + a.q_eps);
#pragma unroll
  for (int s = 0; s < DT; ++s)
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      const int d0 = 32 * s + 16 * part + 8 * h;
      float w[8];
      if (a.q_norm_f32) {
        const f32x4 w0 = *(const f32x4*)((const float*)a.q_norm_w + d0);
        const f32x4 w1 = *(const f32x4*)((const float*)a.q_norm_w + d0 + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = w0[i], w[4 + i] = w1[i];
      } else {
        const bf16x8 w8 = *(const bf16x8*)((const bf16*)a.q_norm_w + d0);
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = (float)w8[i];
      }
      bf16x8& q8 = part ? qf[s].hi : qf[s].lo;
#pragma unroll
      for (int i = 0; i < 8; ++i) q8[i] = (bf16)((float)q8[i] * inv * (1.f + w[i]));
    }
  const bf16* const cs = (const bf16*)a.cosb + (long long)pos * a.rd;
  const bf16* const sn = (const bf16*)a.sinb + (long long)pos * a.rd;
  // rotated slice pairs (s, s + rd / 64), with compile-time slice indices (registers, not scratch)
  switch (a.rd / 64) {
    case 1: rope_pairs<D, 1>(qf, cs, sn, h); break;
    case 2: if constexpr (D / 32 >= 4) rope_pairs<D, 2>(qf, cs, sn, h); break;
    case 3: if constexpr (D / 32 >= 6) rope_pairs<D, 3>(qf, cs, sn, h); break;
    case 4: if constexpr (D / 32 >= 8) rope_pairs<D, 4>(qf, cs, sn, h); break;
    default: break;
  }
}

template <int D>
struct SpSmem {
  // K and V ring stages: four at d = 256 (one phase more of loads in flight, measured 4% faster),
  // three below, where the smaller footprint lets two workgroups share a CU
  static constexpr int NKS = D == 256 ? 4 : 3, NVS = NKS;
  static constexpr int TILE_BYTES = 32 * D * 2;  // one K or V tile of 32 keys
  static constexpr int K_RING = 0, V_RING = NKS * TILE_BYTES;
  // hand-off slot: P fragment (lo halves of the 64 lanes, then hi halves), rescale factor per
  // lane, running max and sum per lane, flags
  static constexpr int P_LO = 0, P_HI = 1024, ALPHA = 2048, MFIN = 2304, LFIN = 2560, FLAGS = 2816;
  static constexpr int SLOT = 2832;
  static constexpr int O_SLOTS = (NKS + NVS) * TILE_BYTES;
  static constexpr int TOTAL = O_SLOTS + 4 * 2 * SLOT;  // [pair][parity]
};
enum { SP_SKIP = 1, SP_RESCALE = 2 };

// TPW: query tiles per workgroup. 4: four consecutive tiles of one query head. 2: two tiles of each
// of two query heads that share a K/V head (even GQA ratios): the workgroup walks the union of the
// key tiles its query tiles see, so fewer consecutive tiles waste fewer phases on tiles only some
// of them see. Every visible tile is walked in the same order either way, so the outputs are the
// same bits.
template <int D, bool BC, int TPW = 4>
__global__ __launch_bounds__(512) void bd_attn_sp_kernel(AttnArgs a) {
  using SM = SpSmem<D>;
  using F = Frag<true>;
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  constexpr int CH = D / 8;          // 16-byte chunks per row
  constexpr int DT = D / 32;         // 32-wide slices of d
  constexpr int RPI = 64 / CH;       // rows per 1 KB wave instruction
  constexpr int IPT = 32 / RPI;      // wave instructions per K (or V) tile
  constexpr int LPW = IPT / 4;       // per wave per tile: the S waves load K, the O waves V
  static_assert(LPW >= 1 && IPT % 4 == 0, "a tile's rows split over four waves");
  static_assert(SM::TOTAL <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) unsigned char smem[SM::TOTAL];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int pair = wave & 3;
  const bool swave = wave < 4;
  const int L = a.L, C = a.C;
  const int Lq = BC ? a.M : L;
  const int Lk = BC ? a.N : L;
  const int qa = BC ? a.q0 : 0;
  const int ntq = (Lq + 31) >> 5;
  static_assert(TPW == 4 || TPW == 2, "query tiles per workgroup");
  constexpr int HPW = 4 / TPW;  // query heads per workgroup
  const int ng = (ntq + TPW - 1) / TPW;
  const int rep = a.Hq / a.Hkv;
  const int nhu = rep / HPW;    // head units per K/V head

  // work unit: longest first (tile group descending), then half, batch, KV head, query heads in group
  constexpr int NH = BC ? 1 : 2;
  const int lin = attn_unit(blockIdx.x, gridDim.x, NH * nhu);
  const int per_g = NH * a.B * a.Hkv * nhu;
  const int g = ng - 1 - lin / per_g;
  int rem = lin % per_g;
  const int qh = BC ? 1 : rem % 2;
  rem /= NH;
  const int hr = rem % nhu;
  rem /= nhu;
  const int hkv = rem % a.Hkv;
  const int b = rem / a.Hkv;
  const int hq = hkv * rep + hr * HPW + pair / TPW;  // this wave pair's query head

  const int g0 = g * (32 * TPW), g1 = min(Lq, g0 + 32 * TPW);
  const int r0 = g0 + (pair % TPW) * 32, r1 = min(Lq, r0 + 32);
  const bool wave_live = r0 < Lq;
  const int qb0 = (qa + r0) / C, qb1 = (qa + max(r0, r1 - 1)) / C;
  const int gqb0 = (qa + g0) / C, gqb1 = (qa + g1 - 1) / C;
  int lo0, hi0, lo1, hi1;
  if (qh == 1) {
    lo0 = hi0 = 0;
    lo1 = 0;
    hi1 = min(Lk, (gqb1 + 1) * C);
  } else {
    lo0 = a.leak ? 0 : gqb0 * C;
    hi0 = min(L, (gqb1 + 1) * C);
    lo1 = 0;
    hi1 = min(L, gqb1 * C);
  }
  const int t0lo = lo0 >> 5, t0hi = (hi0 + 31) >> 5;
  const int t1lo = lo1 >> 5, t1hi = (hi1 + 31) >> 5;
  const int n0 = hi0 > lo0 ? t0hi - t0lo : 0;
  const int n1 = hi1 > lo1 ? t1hi - t1lo : 0;
  const int ntiles = n0 + n1;
  auto tile_pos = [&](int n, int& kh, int& j0) {
    if (n < n1) { kh = 1; j0 = (t1lo + n) * 32; }
    else { kh = 0; j0 = (t0lo + n - n1) * 32; }
  };
  int nbeg = 0, nend = ntiles;
  if constexpr (BC) {
    if (a.ksplit > 1) {
      const int per = (ntiles + a.ksplit - 1) / a.ksplit;
      nbeg = min(ntiles, (int)blockIdx.y * per);
      nend = min(ntiles, nbeg + per);
    }
  }

  const bf16* const qbase = (const bf16*)a.q + b * a.q_sb + (long long)hq * a.q_sh;
  const bf16* const kbase = (const bf16*)a.k + b * a.k_sb + (long long)hkv * a.k_sh;
  const bf16* const vbase = (const bf16*)a.v + b * a.v_sb + (long long)hkv * a.v_sh;

  // Direct load j of this wave's LPW for tile m (K rows by an S wave, V rows by an O wave) into
  // the tile's ring stage. A CU keeps about 32 such 1 KB loads in flight and one wave issues one
  // about every 100-140 cycles (measured), so all eight waves share a tile's loads: the S waves
  // at the start of the phase, the O waves between their products.
  auto stage_one = [&](int m, int j) {
    int kh, j0;
    tile_pos(m, kh, j0);
    const int row0 = (pair * LPW + j) * RPI;
    const int row = row0 + lane / CH;
    const int chunk = (lane % CH) ^ swz_key<D>(row);
    const int key = min(j0 + row, Lk - 1);
    const long long off = (long long)((BC ? 0 : kh * L) + key) * (swave ? a.k_st : a.v_st) + chunk * 8;
    const bf16* src = (swave ? kbase : vbase) + off;
    unsigned char* dst = smem + (swave ? SM::K_RING + (m % SM::NKS) * SM::TILE_BYTES
                                       : SM::V_RING + (m % SM::NVS) * SM::TILE_BYTES) + row0 * (2 * D);
    dma_load16(src, dst);
  };
  auto stage_tile = [&](int m) {
    if (m < nend)
#pragma unroll
      for (int j = 0; j < LPW; ++j) stage_one(m, j);
  };
  auto slot = [&](int n) { return smem + SM::O_SLOTS + (pair * 2 + (n & 1)) * SM::SLOT; };
  constexpr int KD = SM::NKS, VD = SM::NVS - 2;  // load distances of K and V in phases
  static_assert(KD >= 3 && KD <= 4 && VD >= 1 && VD <= 2, "stage counts");
  // wait until at most `tiles` of this wave's tile loads are still in flight
  auto wait_tiles = [&](int tiles) {
    if (tiles >= 2) wait_vmcnt<2 * LPW>();
    else if (tiles == 1) wait_vmcnt<LPW>();
    else wait_vmcnt<0>();
  };

  // Schedule (phase n = the barrier interval of tile n): the S waves form S^T of tile n + 1 and,
  // in the same instruction stream, the softmax of tile n (formed in the phase before), so that
  // the products of one run in the matrix core while the vector unit works on the other; the O
  // waves accumulate tile n - 1. K of tile m is loaded in phase m - KD and read in phase m - 1, V
  // of tile m is loaded in phase m - VD and read in phase m + 1: each stage is reloaded in the
  // phase after its last read.
  // The two roles run separate loops with the same barrier sequence, so that neither holds the
  // other's registers (Q of the S waves, O of the O waves).
  if (swave) {
    // Q^T fragments of the query tile (contiguous d runs)
    F qf[DT];
    const int qrow = min(r0 + l32, Lq - 1);
    {
      const bf16* qp = qbase + (long long)((BC ? 0 : qh * L) + qrow) * a.q_st;
#pragma unroll
      for (int s = 0; s < DT; ++s) {
        qf[s].lo = *(const bf16x8*)(qp + 32 * s + 8 * h);
        qf[s].hi = *(const bf16x8*)(qp + 32 * s + 16 + 8 * h);
      }
    }
    // keys visible to this lane's query in each half: [vlo, vhi) (empty past the last query)
    const int qi = r0 + l32;
    const int qbl = (qa + qi) / C;
    int vlo0, vhi0, vlo1, vhi1;
    if (qh == 1) {
      vlo0 = vhi0 = 0;
      vlo1 = 0;
      vhi1 = min(Lk, (qbl + 1) * C);
    } else {
      vlo0 = a.leak ? 0 : qbl * C;
      vhi0 = min(Lk, (qbl + 1) * C);
      vlo1 = 0;
      vhi1 = min(Lk, qbl * C);
    }
    if (!(wave_live && qi < Lq)) vhi0 = vlo0, vhi1 = vlo1;
    float mrow = -1e30f, lrow = 0.f;  // running max (log2 units) and sum of the query

    auto s_product = [&](int m) {  // S^T = K Q^T of tile m (its K stage)
      const unsigned char* Ks = smem + SM::K_RING + (m % SM::NKS) * SM::TILE_BYTES;
      f32x16 st = zero16();
#pragma unroll
      for (int s = 0; s < DT; ++s) {
        F kf;
        kf.lo = *(const bf16x8*)(Ks + swz_off<D>(l32, 32 * s + 8 * h));
        kf.hi = *(const bf16x8*)(Ks + swz_off<D>(l32, 32 * s + 16 + 8 * h));
        mma32(st, kf, qf[s]);
      }
      return st;
    };
    // phase n: cur holds S^T of tile n; nxt receives S^T of tile n + 1
    auto s_phase = [&](int n, f32x16& cur, f32x16& nxt) {
      stage_tile(n + KD);  // its stage held K of tile n, read in the phase before
      int kh, j0;
      tile_pos(n, kh, j0);
      const int kb0 = j0 / C, kb1 = (min(Lk, j0 + 32) - 1) / C;
      bool any = false, all = false;
      if (wave_live) classify(qh, qb0, qb1, kh, kb0, kb1, a.leak, any, all);
      const bool ragged = (j0 + 32 > Lk) || (r1 - r0 < 32);
      if (!all || ragged) {  // keys this lane's query may not see -> -inf (a tile none may see: all)
        const int lo = kh ? vlo1 : vlo0, hi = kh ? vhi1 : vhi0;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int kj = j0 + rho(v, h);
          cur[v] = (kj >= lo && kj < hi) ? cur[v] : -INFINITY;
        }
      }
      // S^T of tile n + 1 (past the last tile: a stale stage, never used)
      nxt = s_product(n + 1);
      // softmax of tile n, branch-free so that it interleaves with the products above; scores in
      // log2 units, the exponent formed with one rounding (fma of the raw score)
      const float sc = a.scale_log2e;  // > 0 (dispatch): the max of the rounded products is the
      float mx = cur[0];               // rounded product of the max
#pragma unroll
      for (int v = 1; v < 16; ++v) mx = fmaxf(mx, cur[v]);
      mx = halves_max(mx) * sc;
      // lazy rescale (see bd_attn_kernel): the O wave applies alpha before adding this tile;
      // without a rescale alpha = 1 (selected: the hardware 2^0 need not be exactly 1)
      constexpr float RESCALE_LOG2 = 8.f;
      const bool resc = __builtin_amdgcn_ballot_w64(mx > mrow + RESCALE_LOG2) != 0;
      const float mnew = resc ? fmaxf(mrow, mx) : mrow;
      const float alpha = resc ? __builtin_amdgcn_exp2f(mrow - mnew) : 1.f;
      lrow *= alpha;
      mrow = mnew;
      float ps = 0.f;
      f32x16 p;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(cur[v], sc, -mrow));
        ps += p[v];
      }
      ps = halves_sum(ps);
      lrow += ps;
      F pf;
      acc_to_frag(p, pf);
      unsigned char* sl = slot(n);
      *(bf16x8*)(sl + SM::P_LO + 16 * lane) = pf.lo;
      *(bf16x8*)(sl + SM::P_HI + 16 * lane) = pf.hi;
      *(float*)(sl + SM::ALPHA + 4 * lane) = alpha;
      *(float*)(sl + SM::MFIN + 4 * lane) = mrow;  // the last tile's carry the final max and sum
      *(float*)(sl + SM::LFIN + 4 * lane) = lrow;
      *(int*)(sl + SM::FLAGS) = any ? (resc ? SP_RESCALE : 0) : SP_SKIP;  // every lane: one value
      // end of the phase: K of tile n + 2 landed (n + 3 .. n + KD may travel), then the barrier
      wait_tiles(min(KD - 2, max(0, nend - (n + 3))));
      __syncthreads();
    };

    // prologue: K of the first KD tiles, the first two landed; S^T of the first tile
    wait_vmcnt<0>();  // only the direct loads are counted below
#pragma unroll
    for (int i = 0; i < KD; ++i) stage_tile(nbeg + i);
    // the q prologue while the first K tiles travel (its own loads have returned when it ends)
    if constexpr (!BC) {
      if (a.q_norm_w) q_norm_rope<D>(qf, a, qrow, h);  // the row's position within its half
    }
    wait_tiles(min(KD - 2, max(0, nend - (nbeg + 2))));
    __syncthreads();
    f32x16 sa = s_product(nbeg), sb;  // past the last tile: never used
    __syncthreads();  // the first phase restages K of tile nbeg's stage
    for (int n = nbeg; n < nend; n += 2) {
      s_phase(n, sa, sb);
      if (n + 1 < nend) s_phase(n + 1, sb, sa);
    }
    return;
  }

  // ---- O waves: O^T over the whole d (lane = query column), one tile behind
  f32x16 O[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) O[t] = zero16();
  // One phase of an O wave: O^T += V^T P^T for the tile handed over in slot(m) (m < 0: none),
  // after its rescale, with this wave's direct loads of V tile sv (past the last: none) between
  // the d slices.
  auto o_phase = [&](int m, int sv) {
    int fl = SP_SKIP;
    F pf;
    float alpha = 1.f;
    if (m >= 0) {  // the slot's words are read together (P and alpha are unused when skipped)
      const unsigned char* sl = slot(m);
      fl = *(const int*)(sl + SM::FLAGS);
      pf.lo = *(const bf16x8*)(sl + SM::P_LO + 16 * lane);
      pf.hi = *(const bf16x8*)(sl + SM::P_HI + 16 * lane);
      alpha = *(const float*)(sl + SM::ALPHA + 4 * lane);
    }
    if (fl & SP_SKIP) {
      stage_tile(sv);
      return;
    }
    if (fl & SP_RESCALE) {
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) O[t][v] *= alpha;
    }
    const unsigned char* Vs = smem + SM::V_RING + (m % SM::NVS) * SM::TILE_BYTES;
    const int sl4 = lane & 15;
    const int krow = 4 * h + (sl4 >> 2);
    const int dcol = 16 * ((lane >> 4) & 1) + 4 * (sl4 & 3);
    F vf[DT];
    auto vread = [&](int t) {
      bf16x4 r[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        r[q] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(Vs + swz_off<D>(8 * q + krow, 32 * t + dcol)));
      vf[t].lo = __builtin_shufflevector(r[0], r[1], 0, 1, 2, 3, 4, 5, 6, 7);
      vf[t].hi = __builtin_shufflevector(r[2], r[3], 0, 1, 2, 3, 4, 5, 6, 7);
    };
    constexpr int AHEAD = DT < 3 ? DT : 3;  // V^T fragments in flight ahead of the product
#pragma unroll
    for (int t = 0; t < AHEAD; ++t) vread(t);
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      if (t + AHEAD < DT) vread(t + AHEAD);
      mma32(O[t], vf[t], pf);
      if (sv < nend && ((t + 1) * LPW) / DT != (t * LPW) / DT) stage_one(sv, (t * LPW) / DT);
    }
  };
  // prologue: V of the first VD tiles; the S waves' two barriers
#pragma unroll
  for (int i = 0; i < VD; ++i) stage_tile(nbeg + i);
  __syncthreads();
  __syncthreads();
  for (int n = nbeg; n < nend; ++n) {
    // V stage of tile n + VD held tile n - 2, read in the phase before
    o_phase(n > nbeg ? n - 1 : -1, n + VD);
    // end of the phase: V of tile n landed (n + 1 .. n + VD may travel), then the barrier
    wait_tiles(min(VD, max(0, nend - (n + 1))));
    __syncthreads();
  }
  if (nend > nbeg) o_phase(nend - 1, nend);

  const int qi = r0 + l32;
  float mfin = -1e30f, lfin = 0.f;
  if (nend > nbeg) {
    const unsigned char* sl = slot(nend - 1);
    mfin = *(const float*)(sl + SM::MFIN + 4 * lane);
    lfin = *(const float*)(sl + SM::LFIN + 4 * lane);
  }
  if constexpr (BC) {
    if (a.ksplit > 1) {  // partial result of this key share, unnormalised (an empty share: zeros)
      if (wave_live && qi < Lq) {
        const long long prow = (((long long)blockIdx.y * a.B + b) * Lq + qi) * a.Hq + hq;
        float* op = a.opart + prow * D;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            f32x4 o4;
#pragma unroll
            for (int i = 0; i < 4; ++i) o4[i] = O[t][4 * m + i];
            *(f32x4*)(op + 32 * t + 8 * m + 4 * h) = o4;
          }
        if (h == 0) {
          a.mlpart[2 * prow] = mfin;
          a.mlpart[2 * prow + 1] = lfin;
        }
      }
      return;
    }
  }
  if (wave_live && qi < Lq) {
    const float inv = 1.f / lfin;
    const long long orow = BC ? (long long)b * Lq + qi : (long long)b * 2 * L + qh * L + qi;
    bf16* op = (bf16*)a.out + (orow * a.Hq + hq) * a.d;
    // the output gate (gated attention, [hf]:698): bf16(bf16(o) * bf16(sigmoid(gate))), the
    // rounding of the separate elementwise product
    if (a.gate) {
      // every gate value of the row first (in flight together), then the products;
      // sigmoid(x) = 1 / (1 + 2^(-x log2 e)) from the hardware exp2 and reciprocal, rounded to bf16
      const bf16* gp = (const bf16*)a.gate + b * a.g_sb + (long long)(BC ? qi : qh * L + qi) * a.g_st +
                       (long long)hq * a.g_sh;
      bf16x4 g4[DT][4];
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int m = 0; m < 4; ++m) g4[t][m] = *(const bf16x4*)(gp + 32 * t + 8 * m + 4 * h);
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          bf16x4 o4;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float o = (float)(bf16)(O[t][4 * m + i] * inv);
            const float sg = (float)(bf16)__builtin_amdgcn_rcpf(
                1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * (float)g4[t][m][i]));
            o4[i] = (bf16)(o * sg);
          }
          *(bf16x4*)(op + 32 * t + 8 * m + 4 * h) = o4;
        }
    } else {
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          bf16x4 o4;
#pragma unroll
          for (int i = 0; i < 4; ++i) o4[i] = (bf16)(O[t][4 * m + i] * inv);
          *(bf16x4*)(op + 32 * t + 8 * m + 4 * h) = o4;
        }
    }
  }
}

// Merge of the key shares of a split block-causal launch: per (b, query, head) row, with
// M = max_s m_s and w_s = 2^(m_s - M), out = (sum_s w_s O_s) / (sum_s w_s l_s), times sigmoid(gate)
// with the main kernel's rounding when a gate is given (row (b, i, h) of [B, M, Hq, d] at
// b g_sb + i g_st + h g_sh). One thread per four consecutive d.
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ opart,
                                                           const float* __restrict__ mlpart, bf16* __restrict__ out,
                                                           long long rows, int d, int ks, const bf16* __restrict__ gate,
                                                           long long g_sb, int g_st, int g_sh, int M, int Hq) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const int q4 = d / 4;
  if (t >= rows * q4) return;
  const long long row = t / q4;
  const int c = (int)(t % q4) * 4;
  float mx = -1e30f;
  for (int s = 0; s < ks; ++s) mx = fmaxf(mx, mlpart[2 * (s * rows + row)]);
  float l = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < ks; ++s) {
    const float w = __builtin_amdgcn_exp2f(mlpart[2 * (s * rows + row)] - mx);
    l += w * mlpart[2 * (s * rows + row) + 1];
    const f32x4 p = *(const f32x4*)(opart + (s * rows + row) * d + c);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] += w * p[i];
  }
  const float inv = 1.f / l;
  bf16x4 r;
  if (gate) {
    const long long bi = row / Hq;  // b M + i
    const bf16x4 g4 = *(const bf16x4*)(gate + (bi / M) * g_sb + (long long)(bi % M) * g_st +
                                       (long long)(row % Hq) * g_sh + c);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ov = (float)(bf16)(o[i] * inv);
      const float sg = (float)(bf16)__builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * (float)g4[i]));
      r[i] = (bf16)(ov * sg);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = (bf16)(o[i] * inv);
  }
  *(bf16x4*)(out + row * d + c) = r;
}

template <int D, bool BC>
static int launch_attn_sp(const AttnArgs& a, hipStream_t st) {
  const int ntq = ((BC ? a.M : a.L) + 31) / 32;
  // two query heads per workgroup where the GQA ratio is even (complementary-mask mode; measured
  // 911.6 vs 947.2 us at B=2 L=4096 Hq=24 Hkv=4 d=256, bit-identical)
  const bool two = !BC && (a.Hq / a.Hkv) % 2 == 0;
  const int tpw = two ? 2 : 4;
  const int ng = (ntq + tpw - 1) / tpw;
  const long long nblk = (long long)ng * (BC ? 1 : 2) * a.B * a.Hq / (4 / tpw);
  if (nblk > 0x7fffffff) return fail(DLLM_EUNSUPPORTED, "attention: grid too large");
  const int ks = BC && a.ksplit > 1 ? a.ksplit : 1;
  if (two) bd_attn_sp_kernel<D, BC, 2><<<dim3((unsigned)nblk, ks), dim3(512), 0, st>>>(a);
  else bd_attn_sp_kernel<D, BC, 4><<<dim3((unsigned)nblk, ks), dim3(512), 0, st>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "attention launch: %s", hipGetErrorString(e));
  if (ks > 1) {
    const long long rows = (long long)a.B * a.M * a.Hq;
    const long long n = rows * (D / 4);
    attn_combine_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st>>>(
        a.opart, a.mlpart, (bf16*)a.out, rows, D, ks, (const bf16*)a.gate, a.g_sb, a.g_st, a.g_sh, a.M, a.Hq);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(DLLM_ELAUNCH, "attention combine launch: %s", hipGetErrorString(e));
  }
  return DLLM_OK;
}

static bool fits32(long long x) { return x >= -2147483647LL && x <= 2147483647LL; }

// shared by both entry points: vectorisation check and kernel choice
template <bool BC>
static int dispatch_attn(AttnArgs& a, const int64_t* const sts[3], int dtype, hipStream_t st, bool direct_only = false) {
  const int d = a.d;
  const int esz = dtype == DT_BF16 ? 2 : 4;
  const int vel = 16 / esz;
  const int dw = d <= 32 ? 32 : d <= 64 ? 64 : d <= 128 ? 128 : 256;
  bool vec = (d == dw);
  for (int i = 0; i < 3; ++i) vec = vec && (sts[i][0] % vel == 0) && (sts[i][1] % vel == 0) && (sts[i][2] % vel == 0);
  vec = vec && ((uintptr_t)a.q % 16 == 0) && ((uintptr_t)a.k % 16 == 0) && ((uintptr_t)a.v % 16 == 0);
  a.vec = vec;
  if (dtype == DT_BF16) {
    // the direct-load kernel needs whole 16-byte rows of exactly d elements (vectorisable layout)
    // and a positive finite softmax scale
    if (vec && d == dw && dw >= 64 && (a.k_st % 8) == 0 && (a.v_st % 8) == 0 && a.scale_log2e > 0.f &&
        a.scale_log2e < INFINITY) {
      switch (dw) {
        case 64: return launch_attn_sp<64, BC>(a, st);
        case 128: return launch_attn_sp<128, BC>(a, st);
        default: return launch_attn_sp<256, BC>(a, st);
      }
    }
    if (direct_only)
      return fail(DLLM_EUNSUPPORTED, "attention: the gated form needs the direct-load kernel (bf16, d in {64, 128, "
                                     "256}, 16-byte aligned rows of exactly d elements, a positive scale)");
    switch (dw) {
      case 32: return launch_attn<32, true, BC>(a, st);
      case 64: return launch_attn<64, true, BC>(a, st);
      case 128: return launch_attn<128, true, BC>(a, st);
      default: return launch_attn<256, true, BC>(a, st);
    }
  }
  if (direct_only) return fail(DLLM_EUNSUPPORTED, "attention: the gated form is bf16 only");
  if (dtype == DT_F32) {
    switch (dw) {
      case 32: return launch_attn<32, false, BC>(a, st);
      case 64: return launch_attn<64, false, BC>(a, st);
      case 128: return launch_attn<128, false, BC>(a, st);
      default: return launch_attn<256, false, BC>(a, st);
    }
  }
  return fail(DLLM_EUNSUPPORTED, "attention: dtype %d not supported", dtype);
}

static void fill_strides(AttnArgs& a, const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides) {
  a.q_sb = q_strides[0]; a.q_st = (int)q_strides[1]; a.q_sh = (int)q_strides[2];
  a.k_sb = k_strides[0]; a.k_st = (int)k_strides[1]; a.k_sh = (int)k_strides[2];
  a.v_sb = v_strides[0]; a.v_st = (int)v_strides[1]; a.v_sh = (int)v_strides[2];
}

}  // namespace dllm

using namespace dllm;

extern "C" int dllm_bd_attention_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                                     const void* v, const int64_t* v_strides, void* out, int B, int L, int Hq, int Hkv,
                                     int d, int block, float scale, int dtype, int flags, void* stream) {
  if (!q || !k || !v || !out || !q_strides || !k_strides || !v_strides)
    return fail(DLLM_EINVAL, "attention: null pointer");
  if (B <= 0 || L <= 0 || Hq <= 0 || Hkv <= 0 || d <= 0 || block <= 0)
    return fail(DLLM_EINVAL, "attention: bad sizes B=%d L=%d Hq=%d Hkv=%d d=%d block=%d", B, L, Hq, Hkv, d, block);
  if (L % block) return fail(DLLM_EINVAL, "L=%d is not a multiple of block=%d", L, block);
  if (Hq % Hkv) return fail(DLLM_EINVAL, "attention: Hq=%d is not a multiple of Hkv=%d", Hq, Hkv);
  if (d > 256) return fail(DLLM_EUNSUPPORTED, "attention: head_dim %d > 256 not supported", d);
  const int64_t* const sts[3] = {q_strides, k_strides, v_strides};
  const int H[3] = {Hq, Hkv, Hkv};
  for (int i = 0; i < 3; ++i)
    if (!fits32(2LL * L * sts[i][1]) || !fits32((long long)H[i] * sts[i][2]) ||
        !fits32(2LL * L * sts[i][1] + (long long)H[i] * sts[i][2]))
      return fail(DLLM_EUNSUPPORTED, "attention: per-sequence extent exceeds 32-bit element offsets");
  AttnArgs a = {};
  a.q = q; a.k = k; a.v = v; a.out = out;
  fill_strides(a, q_strides, k_strides, v_strides);
  a.B = B; a.L = L; a.Hq = Hq; a.Hkv = Hkv; a.d = d; a.C = block;
  a.leak = flags & 1;
  a.scale_log2e = scale * 1.4426950408889634f;
  return dispatch_attn<false>(a, sts, dtype, (hipStream_t)stream);
}

extern "C" int dllm_bd_attention_gated_supported(int d, int rotary_dim, int dtype) {
  return dtype == DT_BF16 && (d == 64 || d == 128 || d == 256) && rotary_dim >= 0 && rotary_dim % 64 == 0 &&
         rotary_dim <= d;
}

extern "C" int dllm_bd_attention_gated_fwd(const void* q, const int64_t* q_strides, const void* k,
                                           const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                           const void* gate, const int64_t* gate_strides, const void* q_norm_w,
                                           int q_norm_dtype, float q_norm_eps, const void* cos_table,
                                           const void* sin_table, int rotary_dim, void* out, int B, int L, int Hq,
                                           int Hkv, int d, int block, float scale, int dtype, int flags, void* stream) {
  if (!q || !k || !v || !out || !q_strides || !k_strides || !v_strides)
    return fail(DLLM_EINVAL, "gated attention: null pointer");
  if (gate && !gate_strides) return fail(DLLM_EINVAL, "gated attention: gate without strides");
  if (q_norm_w && rotary_dim > 0 && (!cos_table || !sin_table))
    return fail(DLLM_EINVAL, "gated attention: null rotary table");
  if (B <= 0 || L <= 0 || Hq <= 0 || Hkv <= 0 || d <= 0 || block <= 0)
    return fail(DLLM_EINVAL, "gated attention: bad sizes B=%d L=%d Hq=%d Hkv=%d d=%d block=%d", B, L, Hq, Hkv, d, block);
  if (L % block) return fail(DLLM_EINVAL, "L=%d is not a multiple of block=%d", L, block);
  if (Hq % Hkv) return fail(DLLM_EINVAL, "attention: Hq=%d is not a multiple of Hkv=%d", Hq, Hkv);
  if (!dllm_bd_attention_gated_supported(d, q_norm_w ? rotary_dim : 0, dtype))
    return fail(DLLM_EUNSUPPORTED, "gated attention: fused form needs bf16, d in {64, 128, 256} and a rotary_dim "
                "that is a multiple of 64 (d=%d rotary_dim=%d dtype=%d)", d, rotary_dim, dtype);
  if (q_norm_w && q_norm_dtype != DT_BF16 && q_norm_dtype != DT_F32)
    return fail(DLLM_EUNSUPPORTED, "gated attention: q norm weight dtype %d", q_norm_dtype);
  const int64_t* const sts[3] = {q_strides, k_strides, v_strides};
  const int H[3] = {Hq, Hkv, Hkv};
  for (int i = 0; i < 3; ++i)
    if (!fits32(2LL * L * sts[i][1]) || !fits32((long long)H[i] * sts[i][2]) ||
        !fits32(2LL * L * sts[i][1] + (long long)H[i] * sts[i][2]))
      return fail(DLLM_EUNSUPPORTED, "attention: per-sequence extent exceeds 32-bit element offsets");
  if (gate && (!fits32(2LL * L * gate_strides[1] + (long long)Hq * gate_strides[2]) || gate_strides[1] % 4 ||
               gate_strides[2] % 4 || (uintptr_t)gate % 8))
    return fail(DLLM_EUNSUPPORTED, "gated attention: gate rows must be 8-byte aligned with 32-bit extents");
  const uintptr_t al = (uintptr_t)q_norm_w | (uintptr_t)cos_table | (uintptr_t)sin_table;
  if (q_norm_w && (al % 16 || rotary_dim % 8))
    return fail(DLLM_EUNSUPPORTED, "gated attention: norm weight and rotary tables must be 16-byte aligned");
  AttnArgs a = {};
  a.q = q; a.k = k; a.v = v; a.out = out;
  fill_strides(a, q_strides, k_strides, v_strides);
  a.B = B; a.L = L; a.Hq = Hq; a.Hkv = Hkv; a.d = d; a.C = block;
  a.leak = flags & 1;
  a.scale_log2e = scale * 1.4426950408889634f;
  a.q_norm_w = q_norm_w;
  a.q_norm_f32 = q_norm_dtype == DT_F32;
  a.q_eps = q_norm_eps;
  a.cosb = cos_table;
  a.sinb = sin_table;
  a.rd = rotary_dim;
  a.gate = gate;
  if (gate) {
    a.g_sb = gate_strides[0];
    a.g_st = (int)gate_strides[1];
    a.g_sh = (int)gate_strides[2];
  }
  // the fused prologue and epilogue live in the direct-load kernel only: refuse a layout it does not take
  const int esz = 2, vel = 16 / esz;
  bool vec = true;
  for (int i = 0; i < 3; ++i) vec = vec && (sts[i][0] % vel == 0) && (sts[i][1] % vel == 0) && (sts[i][2] % vel == 0);
  vec = vec && ((uintptr_t)q % 16 == 0) && ((uintptr_t)k % 16 == 0) && ((uintptr_t)v % 16 == 0);
  if (!vec || !(a.scale_log2e > 0.f && a.scale_log2e < INFINITY))
    return fail(DLLM_EUNSUPPORTED, "gated attention: q/k/v rows must be 16-byte aligned and the scale positive");
  a.vec = 1;
  switch (d) {
    case 64: return launch_attn_sp<64, false>(a, (hipStream_t)stream);
    case 128: return launch_attn_sp<128, false>(a, (hipStream_t)stream);
    default: return launch_attn_sp<256, false>(a, (hipStream_t)stream);
  }
}

static int block_causal_attention(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                                  const void* v, const int64_t* v_strides, const void* gate,
                                  const int64_t* gate_strides, void* out, int B, int M, int N, int q0, int Hq, int Hkv,
                                  int d, int block, float scale, int dtype, float* workspace, int key_splits,
                                  void* stream) {
  if (!q || !k || !v || !out || !q_strides || !k_strides || !v_strides)
    return fail(DLLM_EINVAL, "block-causal attention: null pointer");
  if (B <= 0 || M <= 0 || N <= 0 || q0 < 0 || Hq <= 0 || Hkv <= 0 || d <= 0 || block <= 0)
    return fail(DLLM_EINVAL, "block-causal attention: bad sizes B=%d M=%d N=%d q0=%d Hq=%d Hkv=%d d=%d block=%d", B,
                M, N, q0, Hq, Hkv, d, block);
  if ((long long)q0 + M > 0x7fffffffLL) return fail(DLLM_EINVAL, "block-causal attention: q0 + M overflows");
  if (key_splits < 1 || key_splits > 64) return fail(DLLM_EINVAL, "block-causal attention: key_splits=%d (1..64)", key_splits);
  if (key_splits > 1 && !workspace) return fail(DLLM_EINVAL, "block-causal attention: key splits need a workspace");
  if (Hq % Hkv) return fail(DLLM_EINVAL, "attention: Hq=%d is not a multiple of Hkv=%d", Hq, Hkv);
  if (d > 256) return fail(DLLM_EUNSUPPORTED, "attention: head_dim %d > 256 not supported", d);
  const int64_t* const sts[3] = {q_strides, k_strides, v_strides};
  const int H[3] = {Hq, Hkv, Hkv};
  const int rows[3] = {M, N, N};
  for (int i = 0; i < 3; ++i)
    if (!fits32((long long)rows[i] * sts[i][1]) || !fits32((long long)H[i] * sts[i][2]) ||
        !fits32((long long)rows[i] * sts[i][1] + (long long)H[i] * sts[i][2]))
      return fail(DLLM_EUNSUPPORTED, "attention: per-sequence extent exceeds 32-bit element offsets");
  if (gate && (!fits32((long long)M * gate_strides[1] + (long long)Hq * gate_strides[2]) || gate_strides[1] % 4 ||
               gate_strides[2] % 4 || gate_strides[0] % 4 || (uintptr_t)gate % 8))
    return fail(DLLM_EUNSUPPORTED, "block-causal attention: gate rows must be 8-byte aligned with 32-bit extents");
  AttnArgs a = {};
  a.q = q; a.k = k; a.v = v; a.out = out;
  fill_strides(a, q_strides, k_strides, v_strides);
  a.B = B; a.L = 0; a.Hq = Hq; a.Hkv = Hkv; a.d = d; a.C = block;
  a.M = M; a.N = N; a.q0 = q0;
  a.ksplit = key_splits;
  a.opart = workspace;
  a.mlpart = workspace ? workspace + (long long)key_splits * B * M * Hq * d : nullptr;
  a.scale_log2e = scale * 1.4426950408889634f;
  a.gate = gate;
  if (gate) {
    a.g_sb = gate_strides[0];
    a.g_st = (int)gate_strides[1];
    a.g_sh = (int)gate_strides[2];
  }
  return dispatch_attn<true>(a, sts, dtype, (hipStream_t)stream, gate != nullptr);
}

extern "C" int dllm_block_causal_attention_fwd(const void* q, const int64_t* q_strides, const void* k,
                                               const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                               void* out, int B, int M, int N, int q0, int Hq, int Hkv, int d,
                                               int block, float scale, int dtype, float* workspace, int key_splits,
                                               void* stream) {
  return block_causal_attention(q, q_strides, k, k_strides, v, v_strides, nullptr, nullptr, out, B, M, N, q0, Hq, Hkv,
                                d, block, scale, dtype, workspace, key_splits, stream);
}

extern "C" int dllm_block_causal_attention_gated_fwd(const void* q, const int64_t* q_strides, const void* k,
                                                     const int64_t* k_strides, const void* v,
                                                     const int64_t* v_strides, const void* gate,
                                                     const int64_t* gate_strides, void* out, int B, int M, int N,
                                                     int q0, int Hq, int Hkv, int d, int block, float scale,
                                                     int dtype, float* workspace, int key_splits, void* stream) {
  if (!gate || !gate_strides) return fail(DLLM_EINVAL, "block-causal attention: null gate");
  return block_causal_attention(q, q_strides, k, k_strides, v, v_strides, gate, gate_strides, out, B, M, N, q0, Hq,
                                Hkv, d, block, scale, dtype, workspace, key_splits, stream);
}
