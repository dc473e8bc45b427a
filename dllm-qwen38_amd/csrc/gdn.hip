// Chunked gated delta rule with per-chunk states and the fused state fork (gfx950 / CDNA4).
//
// One workgroup owns one (sequence b, value head hv, window of DVW value columns) and walks the
// sequence in 32-row tiles. A tile holds `sub` real tokens (sub = gcd(chunk, 32)); the other rows
// are zero, which are exact no-ops of the recurrence (k = q = v = 0, beta = 0, g = 0).
//
// Waves: a set of 4 wavefronts per stream (clean; plus noised in fork mode, 8 waves in total, so
// every SIMD runs one clean and one noised wave and each hides the other's latency).
// Per tile and stream:
//   load    q, k (key head hv / (Hv/Hk): GQA by indexing, no expansion), v, beta, g from the
//           registers prefetched during the previous tile, raw into LDS (bf16: all row-major;
//           the transposed operands come from LDS transpose reads); q and k row norms (DPP
//           reductions); gamma = inclusive scan of g over the tile (DPP).
//   G       K K^T and Q K^T on MFMA; decay/beta masks -> A
//           (fp32), P with the q norms and Dk^-1/2 folded in.
//   T       T = (I + A)^-1 in fp32 by a blocked inverse inside the wave that produced A: 8x8
//           diagonal blocks by forward substitution, then the 8x8 and the 16x16 off-diagonal
//           blocks by products. The MFMA operands T1 = T diag(beta e^gamma / ||k||) and
//           T2 = T diag(beta) are formed from it in registers where they are used.
//   W       W = T1 K (= (I+A)^-1 (beta K^ e^gamma)) on MFMA (bf16: into its own rows; fp32:
//           written over the raw k rows).
//   state   wave u of the clean set: U = T2 V, V' = U - W S, O = e^gamma (Q^ S) + P V',
//           S <- e^gamma_last S + K^T (e^(gamma_last - gamma) V'), snapshot S every chunk;
//           wave u of the noised set: the same O with the noised tile's operands and the clean
//           state before the tile, published by the clean set through LDS.
// The recurrent state S (Dk x 32 columns per clean wave) lives in fp32 MFMA accumulators for the
// whole sequence and is fed back as the B operand directly from the accumulator layout.
#include <type_traits>

#include <atomic>

#include "common.h"

namespace dllm {

struct GdnStream {
  const void* q;
  const void* k;
  const void* v;
  const float* beta;
  const float* g;
  void* out;  // [B, T, Hv, Dv] contiguous
};

struct GdnArgs {
  GdnStream s[2];
  const float* init;  // [B, Hv, Dk, Dv] fp32 or null
  float* states;      // [B, T/chunk, Hv, Dk, Dv] fp32 or null
  long long q_sb, k_sb, v_sb, b_sb, g_sb;  // batch strides (elements)
  int q_st, q_sh, k_st, k_sh, v_st, v_sh, b_st, b_sh, g_st, g_sh;  // token / head strides
  int B, T, Hk, Hv, Dk, Dv;
  int sub;         // real rows per 32-row tile
  int snap_every;  // tiles per chunk
  float scale;     // applied to q after l2norm
  int l2norm;
  int vec_qk;  // q/k rows: 16-byte vector loads (aligned, Dk equal to the kernel width)
  int vec_v;   // v rows: 16-byte vector loads (aligned, Dv a multiple of the column window)
  int spin_limit;  // bounded waits give up (and report through dllm_status) after this many sleeps
  int wait_bias;   // 0; tests set a count the LDS wait never reaches, to exercise the give-up path
  // pipelined fork over a range of blocks: rows and snapshots per sequence of the full out and
  // states tensors (T and T / sub for a whole sequence), and the clean state the range starts
  // from (the snapshot of the block before it, in the states layout; null: zeros)
  int t_rows, snap_rows;
  const float* fork_init;
  // pipelined fork with the v channels' causal conv (width 4) + SiLU in the state waves: the v rows
  // read are the conv's inputs; weights [Hv * Dv, 4] (the v channels' rows; bf16, or fp32 in the
  // kernel's fp32-weight instantiation) and bias [Hv * Dv] of the same dtype, or null. t_first: the
  // sequence row of the launch's first row (the history before sequence row 0 is zero).
  const void* vconv_w;
  const void* vconv_b;
  int t_first;
  // the v channels' conv tails (the clean raw rows before each block, [B * nb, tails_cd, 3] from the
  // first v channel on), or null
  void* vtails;
  int tails_cd;
};

// Linear workgroup id such that consecutive ids run on the same XCD (dispatch is round-robin over
// the 8 XCDs): workgroups sharing a key head then share that XCD's L2.
__device__ __forceinline__ int xcd_linear_id(int bid, int n) {
  const int q = n >> 3, r = n & 7, x = bid & 7, i = bid >> 3;
  return (x < r) ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
}

// Returns x unchanged but opaque to the optimiser, so that uniform addresses derived from it are
// computed where they are used instead of being hoisted out of the tile loop (and spilled).
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+s"(x));
  return x;
}
// The same for a per-lane value: comparisons against it are evaluated where they are used instead
// of being hoisted out of the tile loop as lane masks held in (spilled) scalar registers.
__device__ __forceinline__ int opaque_v(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// DPP move; lanes whose source is outside the row read 0 (bound_ctrl).
template <int CTRL> __device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Sum over each aligned group of 8 lanes, returned to all 8 (DPP: no LDS round trip). The three
// steps are quad_perm [1,0,3,2], quad_perm [2,3,0,1] and row_half_mirror.
__device__ __forceinline__ float dpp_sum8(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x141, 0xF, 0xF, true));
  return x;
}

template <int DK, int DVW, bool BF16, bool FORK>
struct GdnSmem {
  using OpT = typename std::conditional<BF16, bf16, float>::type;
  static constexpr int NS = FORK ? 2 : 1;
  static constexpr int KT = DK / 32;
  static constexpr int NSL = DVW / 32;
  static constexpr int QROW = DK + (BF16 ? 8 : 4);  // [32][DK] row stride (elements)
  static constexpr int TROW = 36;                    // [.][32] row stride (elements)
  static constexpr int O_QH = 0;
  static constexpr int O_KH = O_QH + 32 * QROW * (int)sizeof(OpT);
  static constexpr int O_KT = O_KH + 32 * QROW * (int)sizeof(OpT);
  static constexpr int O_VT = O_KT + DK * TROW * (int)sizeof(OpT);
  static constexpr int O_P = O_VT + DVW * TROW * (int)sizeof(OpT);
  static constexpr int O_AF = O_P + 32 * TROW * (int)sizeof(OpT);
  static constexpr int FROW = 36;  // fp32 [32][32] scratch row stride (16-byte aligned rows)
  static constexpr int O_TF = O_AF + 32 * FROW * 4;
  static constexpr int O_YF = O_TF + 32 * FROW * 4;
  static constexpr int O_VEC = O_YF + 16 * 20 * 4;  // nine per-row vectors of 32 floats
  static constexpr int STREAM_BYTES = ((O_VEC + 9 * 32 * 4) + 15) & ~15;
  // bf16 keeps k and v row-major (transposed operands come from LDS transpose reads): the two
  // transposed regions hold W rows [32][QROW] and v rows [32][VROW] instead
  static constexpr int VROW = DVW + 8;
  static_assert(!BF16 || 32 * QROW <= DK * TROW, "W rows must fit the k-transpose region");
  static_assert(!BF16 || 32 * VROW <= DVW * TROW, "v rows must fit the v-transpose region");
  static constexpr int FRAG_BYTES = 16 * (int)sizeof(OpT);
  // state operand fragments published by the clean set for the noised set: [NSL][KT][64 lanes]
  static constexpr int O_SB = NS * STREAM_BYTES;
  static constexpr int SB_BYTES = FORK ? NSL * KT * 64 * FRAG_BYTES : 0;
  static constexpr int TOTAL = O_SB + SB_BYTES;
};

// Two runs of N/2 elements of a row into 16-byte vector registers of the raw input dtype.
// `valid0/1` elements of each run are in range, the rest are zero. When a run is shorter than one
// vector the two runs are contiguous (src1 == src0 + N/2) and load as one vector.
template <typename V, typename OpT, int N>
__device__ __forceinline__ void load_runs(V* dst, const OpT* src0, const OpT* src1, bool vec, int valid0,
                                          int valid1) {
  constexpr int EPV = 16 / (int)sizeof(OpT);
  constexpr int H = N / 2;
  if constexpr (H >= EPV) {
    constexpr int NV = H / EPV;  // vectors per run
    if (vec) {  // uniform: every lane's runs are in range (callers clamp rows), no divergence
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        dst[i] = *(const V*)(src0 + i * EPV);
        dst[NV + i] = *(const V*)(src1 + i * EPV);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
          dst[i][e] = (i * EPV + e < valid0) ? src0[i * EPV + e] : from_f32<OpT>(0.f);
          dst[NV + i][e] = (i * EPV + e < valid1) ? src1[i * EPV + e] : from_f32<OpT>(0.f);
        }
    }
  } else {
    static_assert(N == EPV, "a short row segment must be exactly one vector");
    if (vec) {
      dst[0] = *(const V*)src0;
    } else {
#pragma unroll
      for (int e = 0; e < N; ++e)
        dst[0][e] = ((e < H) ? (e < valid0) : (e - H < valid1)) ? src0[e] : from_f32<OpT>(0.f);
    }
  }
}

template <int DK, int DVW, bool BF16, bool FORK>
__global__ __launch_bounds__(FORK ? 512 : 256) void gdn_chunk_kernel(GdnArgs a) {
  using SM = GdnSmem<DK, DVW, BF16, FORK>;
  using OpT = typename SM::OpT;
  using F = Frag<BF16>;
  constexpr int KT = SM::KT;
  constexpr int NSL = SM::NSL;
  constexpr int QROW = SM::QROW;
  constexpr int TROW = SM::TROW;
  constexpr int FROW = SM::FROW;
  constexpr float LOG2E = 1.4426950408889634f;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SM::TOTAL];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform values live in SGPRs
  const int lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int set = FORK ? (wave >> 2) : 0;  // stream of this wave's set
  const int u = wave & 3;                  // wave within the set
  const int ts = tid & 255;                // thread within the set

  const int nwin = (a.Dv + DVW - 1) / DVW;
  const int lin = xcd_linear_id(blockIdx.x, gridDim.x);
  const int win = lin % nwin;
  const int hv = (lin / nwin) % a.Hv;
  const int b = lin / (nwin * a.Hv);
  const int hk = hv / (a.Hv / a.Hk);
  const int col0 = win * DVW;
  const int ntiles = a.T / a.sub;
  const int nsnap = a.T / (a.sub * a.snap_every);

  unsigned char* sbase = smem + set * SM::STREAM_BYTES;
  OpT* const QH = (OpT*)(sbase + SM::O_QH);    // raw q rows            [32][DK]
  OpT* const KH = (OpT*)(sbase + SM::O_KH);    // raw k rows, then W    [32][DK]
  OpT* const KTr = (OpT*)(sbase + SM::O_KT);   // fp32: raw k transposed [DK][32]
  OpT* const VT = (OpT*)(sbase + SM::O_VT);    // fp32: raw v transposed [DVW][32]
  OpT* const WH = KTr;                         // bf16: W rows           [32][QROW]
  OpT* const VH = VT;                          // bf16: raw v rows       [32][VROW]
  constexpr int VROW = SM::VROW;
  OpT* const PP = (OpT*)(sbase + SM::O_P);     // P with q row norms    [32][32]
  float* const AF = (float*)(sbase + SM::O_AF);
  float* const TF = (float*)(sbase + SM::O_TF);
  float* const YF = (float*)(sbase + SM::O_YF);
  float* const GAML = (float*)(sbase + SM::O_VEC);  // cumulative decay, log2 units
  float* const BET = GAML + 32;                     // beta
  float* const EG = GAML + 64;                      // e^gamma
  float* const EGL = GAML + 96;                     // e^(gamma_last - gamma)
  float* const RNK = GAML + 128;                    // 1/||k|| (1 without l2norm)
  float* const RNQ = GAML + 160;                    // scale/||q||
  float* const EGQ = GAML + 192;                    // e^gamma scale/||q||
  float* const EGLK = GAML + 224;                   // e^(gamma_last - gamma)/||k||
  float* const BER = GAML + 256;                    // beta e^gamma/||k|| (column scale of T1)
  auto SBUF = [&](int sl, int kt) { return (F*)(smem + SM::O_SB) + ((sl * KT + kt) * 64 + lane); };

  // this set's stream: base pointers at (b, head)
  const GdnStream& st = a.s[set];
  const OpT* const qb = (const OpT*)st.q + b * a.q_sb + (long long)hk * a.q_sh;
  const OpT* const kb = (const OpT*)st.k + b * a.k_sb + (long long)hk * a.k_sh;
  const OpT* const vb = (const OpT*)st.v + b * a.v_sb + (long long)hv * a.v_sh;
  const float* const betab = st.beta + b * a.b_sb + (long long)hv * a.b_sh;
  const float* const gb = st.g + b * a.g_sb + (long long)hv * a.g_sh;

  // state-phase role: wave u of the set owns value columns [col0 + 32u, col0 + 32u + 32)
  const bool state_wave = u < NSL;
  const int scol0 = col0 + u * 32;  // wave-uniform
  const bool slice_full = scol0 + 32 <= a.Dv;
  const bool col_ok = scol0 + l32 < a.Dv;

  f32x16 S[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) S[t] = zero16();
  if (set == 0 && state_wave && a.init && col_ok) {
    const float* src = a.init + ((long long)(b * a.Hv + hv) * a.Dk) * a.Dv + scol0 + l32;
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int dk = 32 * t + rho(v, h);
        if (dk < a.Dk) S[t][v] = src[(long long)dk * a.Dv];
      }
  }

  // Raw inputs of one tile, in registers so that the next tile's global loads travel while the
  // current tile computes. Thread (row lr, segment lseg) holds two runs of its row: q/k columns
  // [NE/2*lseg, +NE/2) and [DK/2 + NE/2*lseg, +NE/2), v columns likewise in the DVW window (two
  // runs per thread keep the transposed LDS writes nearly conflict-free).
  constexpr int NE = DK / 8;   // q/k elements per thread
  constexpr int NV = DVW / 8;  // v elements per thread
  constexpr int EPV = 16 / (int)sizeof(OpT);
  using V16 = typename std::conditional<BF16, bf16x8, f32x4>::type;
  V16 rq[NE / EPV], rk[NE / EPV], rv[NV / EPV];
  float rg = 0.f, rb = 0.f;
  const int lr = ts >> 3, lseg = ts & 7;
  const bool lreal = lr < a.sub;  // rows >= sub are zero padding (loaded from row 0, zeroed on use)
  constexpr bool TWO_QK = (NE / 2) >= EPV;  // else one contiguous run of NE elements
  constexpr bool TWO_V = (NV / 2) >= EPV;
  const int qe0 = TWO_QK ? lseg * (NE / 2) : lseg * NE;
  const int qe1 = TWO_QK ? DK / 2 + lseg * (NE / 2) : qe0 + NE / 2;
  const int ve0 = TWO_V ? lseg * (NV / 2) : lseg * NV;
  const int ve1 = TWO_V ? DVW / 2 + lseg * (NV / 2) : ve0 + NV / 2;
  auto issue_loads = [&](int t0) {
    const int tok = t0 + (lreal ? lr : 0);
    const int vq0 = lreal ? max(0, min(NE / 2, a.Dk - qe0)) : 0;
    const int vq1 = lreal ? max(0, min(NE / 2, a.Dk - qe1)) : 0;
    const int vv0 = lreal ? max(0, min(NV / 2, a.Dv - col0 - ve0)) : 0;
    const int vv1 = lreal ? max(0, min(NV / 2, a.Dv - col0 - ve1)) : 0;
    const OpT* qr = qb + tok * a.q_st;
    const OpT* kr = kb + tok * a.k_st;
    const OpT* vr = vb + tok * a.v_st + col0;
    load_runs<V16, OpT, NE>(rq, qr + qe0, qr + qe1, a.vec_qk, vq0, vq1);
    load_runs<V16, OpT, NE>(rk, kr + qe0, kr + qe1, a.vec_qk, vq0, vq1);
    load_runs<V16, OpT, NV>(rv, vr + ve0, vr + ve1, a.vec_v, vv0, vv1);
    if (u == 0 && h == 0 && l32 < a.sub) {
      rg = gb[(t0 + l32) * a.g_st];
      rb = betab[(t0 + l32) * a.b_st];
    } else {
      rg = 0.f;
      rb = 0.f;
    }
  };
  issue_loads(0);
  // The waits below keep loads and stores from being in flight together at the points where the
  // prefetched registers are read: with both kinds pending the compiler must wait for every
  // outstanding store (vmcnt(0)) before using a loaded value.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): nothing in flight at the loop head
  const V16 vzero = {};

  for (int c = 0; c < ntiles; ++c) {
    const int t0 = c * a.sub;
    const int lo = opaque_v(l32), ho = opaque_v(h);  // lane indices for masks (see opaque_v)
    __syncthreads();  // the previous tile's state phase is done with every LDS operand

    // ------------------------------------------------------------------ load phase (registers -> LDS)
    // Raw q, k, v are stored as loaded (exact); the l2 norms are applied as row/column scalings
    // of the products. Padding rows store zeros.
    {
      V16 xq[NE / EPV], xk[NE / EPV], xv[NV / EPV];
#pragma unroll
      for (int i = 0; i < NE / EPV; ++i) {
        xq[i] = lreal ? rq[i] : vzero;
        xk[i] = lreal ? rk[i] : vzero;
      }
#pragma unroll
      for (int i = 0; i < NV / EPV; ++i) xv[i] = lreal ? rv[i] : vzero;
      constexpr int HV = TWO_QK ? NE / 2 / EPV : 1;  // vectors per q/k run (single run: 1)
      if constexpr (TWO_QK) {
#pragma unroll
        for (int i = 0; i < HV; ++i) {
          *(V16*)(QH + lr * QROW + qe0 + i * EPV) = xq[i];
          *(V16*)(QH + lr * QROW + qe1 + i * EPV) = xq[HV + i];
          *(V16*)(KH + lr * QROW + qe0 + i * EPV) = xk[i];
          *(V16*)(KH + lr * QROW + qe1 + i * EPV) = xk[HV + i];
        }
      } else {
        *(V16*)(QH + lr * QROW + qe0) = xq[0];
        *(V16*)(KH + lr * QROW + qe0) = xk[0];
      }
      if constexpr (BF16) {  // v rows as loaded: the transposed operands come from transpose reads
        if constexpr (TWO_V) {
          constexpr int HVV = NV / 2 / EPV;
#pragma unroll
          for (int i = 0; i < HVV; ++i) {
            *(V16*)(VH + lr * VROW + ve0 + i * EPV) = xv[i];
            *(V16*)(VH + lr * VROW + ve1 + i * EPV) = xv[HVV + i];
          }
        } else {
          *(V16*)(VH + lr * VROW + ve0) = xv[0];
        }
      } else {
#pragma unroll
        for (int i = 0; i < NE / 2; ++i) {
          KTr[(qe0 + i) * TROW + lr] = xk[i / EPV][i % EPV];
          KTr[(qe1 + i) * TROW + lr] = xk[(NE / 2 + i) / EPV][(NE / 2 + i) % EPV];
        }
#pragma unroll
        for (int i = 0; i < NV / 2; ++i) {
          VT[(ve0 + i) * TROW + lr] = xv[i / EPV][i % EPV];
          VT[(ve1 + i) * TROW + lr] = xv[(NV / 2 + i) / EPV][(NV / 2 + i) % EPV];
        }
      }
      // q and k row norms: fp32 sums of squares of the row (DPP reductions over its 8 threads),
      // as the reference's l2norm; the G phase then needs no round trip for them
      float ss = 0.f, sk = 0.f;
#pragma unroll
      for (int i = 0; i < NE; ++i) {
        const float x = to_f32(xq[i / EPV][i % EPV]);
        const float y = to_f32(xk[i / EPV][i % EPV]);
        ss = __builtin_fmaf(x, x, ss);
        sk = __builtin_fmaf(y, y, sk);
      }
      ss = dpp_sum8(ss);
      sk = dpp_sum8(sk);
      if (lseg == 0) {
        RNQ[lr] = a.l2norm ? a.scale * rsqrtf(ss + 1e-6f) : a.scale;
        RNK[lr] = a.l2norm ? rsqrtf(sk + 1e-6f) : 1.f;
      }
      // beta, g and the cumulative decay (inclusive scan over the tile's rows), one wave per set:
      // lanes 0..31 hold g of rows 0..31 (zero for padding rows and for lanes 32..63); scan
      // within each 16-lane DPP row, then carry row 0's total into row 1 (row_bcast:15)
      if (u == 0) {
        float x = rg;
        x += dpp_mov<0x111>(x);  // row_shr:1
        x += dpp_mov<0x112>(x);  // row_shr:2
        x += dpp_mov<0x114>(x);  // row_shr:4
        x += dpp_mov<0x118>(x);  // row_shr:8
        x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x142, 0xA, 0xF, false));
        const float gam = x;
        const float gall = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 31));
        if (h == 0) {
          GAML[l32] = gam * LOG2E;
          BET[l32] = rb;
          EG[l32] = __builtin_amdgcn_exp2f(gam * LOG2E);
          EGL[l32] = __builtin_amdgcn_exp2f((gall - gam) * LOG2E);
        }
      }
      // the clean set publishes the state before this tile for the noised set
      if constexpr (FORK) {
        if (set == 0 && state_wave) {
#pragma unroll
          for (int t = 0; t < KT; ++t) {
            F f;
            acc_to_frag(S[t], f);
            *SBUF(u, t) = f;
          }
        }
      }
    }
    __syncthreads();
    if (c + 1 < ntiles) issue_loads(t0 + a.sub);  // next tile's inputs travel during this tile

    // ------------------------------------------------------------------ G phase + diagonal blocks of T
    // (every step issues all of its LDS reads before computing: one LDS round trip per step)
    {
      // K K^T (+ A and the blocked inverse T) on waves 0 / 5, Q K^T on waves 2 / 7:
      // four different SIMDs in fork mode
      const bool isG = (u == (set == 0 ? 0 : 1));
      const bool isQK = (u == (set == 0 ? 2 : 3));
      if (isG || isQK) {
        f32x16 acc = zero16();
        f32x4 gam4[4];
        if (isG) {  // K K^T: one operand read serves both sides
          F fa[KT];
#pragma unroll
          for (int kt = 0; kt < KT; ++kt) lds_frag(KH + l32 * QROW + kt * 32, h, fa[kt]);
#pragma unroll
          for (int m = 0; m < 4; ++m) gam4[m] = *(const f32x4*)(GAML + 8 * m + 4 * h);
#pragma unroll
          for (int kt = 0; kt < KT; ++kt) mma32(acc, fa[kt], fa[kt]);
          // issue every operand read before the MFMA chain (one LDS round trip, not one per slice)
          __builtin_amdgcn_sched_group_barrier(0x100, 2 * KT + 4, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 2 * KT, 0);
        } else {
          F fa[KT], fb[KT];
#pragma unroll
          for (int kt = 0; kt < KT; ++kt) {
            lds_frag(QH + l32 * QROW + kt * 32, h, fa[kt]);
            lds_frag(KH + l32 * QROW + kt * 32, h, fb[kt]);
          }
#pragma unroll
          for (int m = 0; m < 4; ++m) gam4[m] = *(const f32x4*)(GAML + 8 * m + 4 * h);
#pragma unroll
          for (int kt = 0; kt < KT; ++kt) mma32(acc, fa[kt], fb[kt]);
          __builtin_amdgcn_sched_group_barrier(0x100, 4 * KT + 4, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 2 * KT, 0);
        }
        const float gj = GAML[l32];
        if (isG) {
          f32x4 bet4[4], rnk4[4];
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            bet4[m] = *(const f32x4*)(BET + 8 * m + 4 * h);
            rnk4[m] = *(const f32x4*)(RNK + 8 * m + 4 * h);
          }
          const float rj = RNK[l32];
          const float eglj = EGL[l32];
#pragma unroll
          for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int i = 8 * m + 4 * h + e;
              const float val = (bet4[m][e] * rnk4[m][e] * rj) * acc[4 * m + e] *
                                __builtin_amdgcn_exp2f(gam4[m][e] - gj);
              AF[i * FROW + l32] = (lo < 8 * m + 4 * ho + e) ? val : 0.f;
            }
          if (h == 0) EGLK[l32] = eglj * rj;
          wave_lds_sync();
          // level 0: four 8x8 diagonal blocks, one column per lane (lanes 0..31); lanes of odd
          // blocks also clear the block above (read as zero by level 2)
          if (h == 0) {
            const int bb = l32 >> 3, cc = lo & 7, o = 8 * bb;
            f32x4 ar[8][2];
#pragma unroll
            for (int i = 1; i < 8; ++i) {
              ar[i][0] = *(const f32x4*)(AF + (o + i) * FROW + o);
              ar[i][1] = *(const f32x4*)(AF + (o + i) * FROW + o + 4);
            }
            float x[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = (i == cc) ? 1.f : 0.f;
#pragma unroll
            for (int i = 1; i < 8; ++i) {
              float sacc = 0.f;
#pragma unroll
              for (int j = 0; j < i; ++j) sacc = __builtin_fmaf(ar[i][j >> 2][j & 3], x[j], sacc);
              if (i > cc) x[i] = -sacc;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) TF[(o + i) * FROW + o + cc] = x[i];
            if (bb & 1) {
#pragma unroll
              for (int i = 0; i < 8; ++i) TF[(o - 8 + i) * FROW + o + cc] = 0.f;
            }
          }
          wave_lds_sync();
          // level 1: T[m+1][m] = -D[m+1] (A[m+1][m] D[m]) for the three sub-diagonal 8x8 blocks
          {
            const int ii = lane >> 3, jj = lane & 7;
            f32x4 arow[3][2];
            float dcol[3][8];
#pragma unroll
            for (int m = 0; m < 3; ++m) {
              arow[m][0] = *(const f32x4*)(AF + (8 * (m + 1) + ii) * FROW + 8 * m);
              arow[m][1] = *(const f32x4*)(AF + (8 * (m + 1) + ii) * FROW + 8 * m + 4);
#pragma unroll
              for (int kk = 0; kk < 8; ++kk) dcol[m][kk] = TF[(8 * m + kk) * FROW + 8 * m + jj];
            }
#pragma unroll
            for (int m = 0; m < 3; ++m) {
              float sacc = 0.f;
#pragma unroll
              for (int kk = 0; kk < 8; ++kk) sacc = __builtin_fmaf(arow[m][kk >> 2][kk & 3], dcol[m][kk], sacc);
              YF[m * 64 + ii * 8 + jj] = sacc;
            }
            wave_lds_sync();
            f32x4 drow[3][2];
            float ycol[3][8];
#pragma unroll
            for (int m = 0; m < 3; ++m) {
              drow[m][0] = *(const f32x4*)(TF + (8 * (m + 1) + ii) * FROW + 8 * (m + 1));
              drow[m][1] = *(const f32x4*)(TF + (8 * (m + 1) + ii) * FROW + 8 * (m + 1) + 4);
#pragma unroll
              for (int kk = 0; kk < 8; ++kk) ycol[m][kk] = YF[m * 64 + kk * 8 + jj];
            }
#pragma unroll
            for (int m = 0; m < 3; ++m) {
              float sacc = 0.f;
#pragma unroll
              for (int kk = 0; kk < 8; ++kk) sacc = __builtin_fmaf(drow[m][kk >> 2][kk & 3], ycol[m][kk], sacc);
              TF[(8 * (m + 1) + ii) * FROW + 8 * m + jj] = -sacc;
            }
          }
          wave_lds_sync();
          // level 2 (this wave): T[16:32][0:16] = -T22 (A21 T11), lane -> row 16 + i2, columns j2..j2+3;
          // every other entry of the lower triangle is final in TF after levels 0 and 1
          {
            const int i2 = lane >> 2, j2 = (lane & 3) * 4;
            f32x4 arow[4], tcol[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) arow[q] = *(const f32x4*)(AF + (16 + i2) * FROW + 4 * q);
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) tcol[kk] = *(const f32x4*)(TF + kk * FROW + j2);
            f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < 16; ++kk)
#pragma unroll
              for (int e = 0; e < 4; ++e) y[e] = __builtin_fmaf(arow[kk >> 2][kk & 3], tcol[kk][e], y[e]);
            *(f32x4*)(YF + i2 * 20 + j2) = y;
            wave_lds_sync();
            f32x4 trow[4], ycol[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) trow[q] = *(const f32x4*)(TF + (16 + i2) * FROW + 16 + 4 * q);
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) ycol[kk] = *(const f32x4*)(YF + kk * 20 + j2);
            f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < 16; ++kk)
#pragma unroll
              for (int e = 0; e < 4; ++e) z[e] = __builtin_fmaf(trow[kk >> 2][kk & 3], ycol[kk][e], z[e]);
            *(f32x4*)(TF + (16 + i2) * FROW + j2) = -z;
          }
          if (h == 0) BER[l32] = BET[l32] * EG[l32] * RNK[l32];
        } else {
          f32x4 rnq4[4];
#pragma unroll
          for (int m = 0; m < 4; ++m) rnq4[m] = *(const f32x4*)(RNQ + 8 * m + 4 * h);
          const float egj = EG[l32], rqj = RNQ[l32];
#pragma unroll
          for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int i = 8 * m + 4 * h + e;
              const float val = rnq4[m][e] * acc[4 * m + e] * __builtin_amdgcn_exp2f(gam4[m][e] - gj);
              PP[i * TROW + l32] = from_f32<OpT>((lo <= 8 * m + 4 * ho + e) ? val : 0.f);
            }
          if (h == 0) EGQ[l32] = egj * rqj;
        }
      }
    }
    __syncthreads();

    // T operand fragments, built from the fp32 T (lower triangle, diagonal included) with a
    // per-column scale: lane = row l32, columns rho(v, h)
    auto t_frag = [&](const float* colscale, F& f) {
      f32x16 tv;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const f32x4 t4 = *(const f32x4*)(TF + l32 * FROW + 8 * m + 4 * h);
        const f32x4 c4 = *(const f32x4*)(colscale + 8 * m + 4 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) tv[4 * m + e] = (8 * m + 4 * ho + e <= lo) ? t4[e] * c4[e] : 0.f;
      }
      acc_to_frag(tv, f);
    };

    // ------------------------------------------------------------------ W phase: W = T1 K_raw
    if (u < KT) {
      const int kt = u;
      F fa, fb;
      t_frag(BER, fa);  // T1 = T diag(beta e^gamma / ||k||)
      if constexpr (BF16) {
        lds_frag_tr(KH + kt * 32, QROW, lane, fb);
      } else {
        lds_frag(KTr + (kt * 32 + l32) * TROW, h, fb);
      }
      f32x16 acc = zero16();
      mma32(acc, fa, fb);
      // bf16: W gets its own rows (raw k stays for the state update); fp32: raw k is dead
      OpT* const Wd = BF16 ? WH : KH;
#pragma unroll
      for (int v = 0; v < 16; ++v) Wd[rho(v, h) * QROW + kt * 32 + l32] = from_f32<OpT>(acc[v]);
    }
    __syncthreads();

    // ------------------------------------------------------------------ state phase
    if (state_wave) {
      f32x16 accU = zero16(), accWS = zero16(), accQS = zero16();
      {
        F fa, fb;
        t_frag(BET, fa);  // T2 = T diag(beta)
        if constexpr (BF16) {
          lds_frag_tr(VH + u * 32, VROW, lane, fb);
        } else {
          lds_frag(VT + (u * 32 + l32) * TROW, h, fb);
        }
        mma32(accU, fa, fb);
      }
      constexpr int KH2 = KT >= 2 ? KT / 2 : 1;  // fragment reads in batches of KH2 K-slices
#pragma unroll
      for (int k0 = 0; k0 < KT; k0 += KH2) {
        F fw[KH2], fq[KH2], sx[KH2];
#pragma unroll
        for (int q = 0; q < KH2; ++q) {
          lds_frag((BF16 ? WH : KH) + l32 * QROW + (k0 + q) * 32, h, fw[q]);
          lds_frag(QH + l32 * QROW + (k0 + q) * 32, h, fq[q]);
          if constexpr (FORK) {
            sx[q] = *SBUF(u, k0 + q);
          } else {
            acc_to_frag(S[k0 + q], sx[q]);
          }
        }
#pragma unroll
        for (int q = 0; q < KH2; ++q) {
          mma32(accWS, fw[q], sx[q]);
          mma32(accQS, fq[q], sx[q]);
        }
      }
      // O = diag(e^gamma scale/||q||) Q_raw S + P (V' / ||k||)
      f32x16 vn, vk;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const f32x4 egq = *(const f32x4*)(EGQ + 8 * m + 4 * h);
        const f32x4 rnk = *(const f32x4*)(RNK + 8 * m + 4 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int v = 4 * m + e;
          vn[v] = accU[v] - accWS[v];
          vk[v] = vn[v] * rnk[e];
          accQS[v] *= egq[e];
        }
      }
      {
        F fv, fp;
        acc_to_frag(vk, fv);
        lds_frag(PP + l32 * TROW, h, fp);
        mma32(accQS, fp, fv);
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the next tile's prefetch has landed
      // output rows of the real tokens: uniform row bases, one 32-bit lane offset
      {
        const int rs = opaque(a.Hv * a.Dv);  // token stride of out
        OpT* ob = (OpT*)st.out + ((long long)b * a.T + t0) * rs + (long long)hv * a.Dv + scol0;
        const unsigned lo = (unsigned)(4 * h * rs + l32);
        if (a.sub == 32 && slice_full) {
#pragma unroll
          for (int v = 0; v < 16; ++v) (ob + (((v >> 2) << 3) + (v & 3)) * rs)[lo] = from_f32<OpT>(accQS[v]);
        } else if (col_ok) {
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int ru = ((v >> 2) << 3) + (v & 3);  // row = ru + 4h
            if (ru + 4 * h < a.sub) (ob + ru * rs)[lo] = from_f32<OpT>(accQS[v]);
          }
        }
      }
      if (set == 0) {
        // S <- e^gamma_last S + K_raw^T (e^(gamma_last - gamma) / ||k|| V')
        const float lam = EG[31];
        f32x16 vd;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const f32x4 eglk = *(const f32x4*)(EGLK + 8 * m + 4 * h);
#pragma unroll
          for (int e = 0; e < 4; ++e) vd[4 * m + e] = vn[4 * m + e] * eglk[e];
        }
        F fd;
        acc_to_frag(vd, fd);
        F fk[KT];
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          if constexpr (BF16) {
            lds_frag_tr(KH + kt * 32, QROW, lane, fk[kt]);
          } else {
            lds_frag(KTr + (kt * 32 + l32) * TROW, h, fk[kt]);
          }
        }
        // state snapshot after every snap_every tiles; for a full head (compile-time row stride)
        // each K slice is stored as soon as its update is issued
        const bool snap = a.states && ((c + 1) % a.snap_every) == 0;
        const int dv = opaque(a.Dv);
        const bool snap_fast = snap && a.Dk == DK && dv == DVW;
        float* const sb = snap ? a.states + (((long long)b * nsnap + ((c + 1) / a.snap_every - 1)) * a.Hv + hv) *
                                                (long long)a.Dk * a.Dv + scol0
                               : nullptr;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
          for (int v = 0; v < 16; ++v) S[kt][v] *= lam;
          mma32(S[kt], fk[kt], fd);
          if (snap_fast) {
            float* lp = sb + 4 * h * DVW + l32;
#pragma unroll
            for (int v = 0; v < 16; ++v)
              __builtin_nontemporal_store(S[kt][v], lp + (32 * kt + ((v >> 2) << 3) + (v & 3)) * DVW);
          }
        }
        if (snap && !snap_fast) {
          if (col_ok) {
            const unsigned lo = (unsigned)(4 * h * dv + l32);
#pragma unroll
            for (int kt = 0; kt < KT; ++kt)
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const int du = 32 * kt + ((v >> 2) << 3) + (v & 3);  // dk = du + 4h
                if (du + 4 * h < a.Dk) __builtin_nontemporal_store(S[kt][v], (sb + (long long)du * dv) + lo);
              }
          }
        }
      }
    }
  }
}

// ============================================================================================
// Pipelined state fork (bf16, Dk = Dv = 128, one workgroup per (sequence, value head)).
//
// The recurrence S <- e^gamma_last S + K~^T V', V' = U - T1 K S, is the only sequential
// dependency of a tile; the Gram products, the inverse T = (I + A)^-1 and its scaled operands
// T1, T2 (U = T2 V), and P = mask(Q K^T) depend on the tile's inputs alone. They are formed one
// tile AHEAD, beside the state work of the current tile:
//   waves 0-3 (state waves) each own 32 value columns of BOTH streams. They hold the clean state of
//            their columns in MFMA accumulators and, per tile, form K S and Q S of both streams
//            from it, then V' = T2 V - T1 (K S) (W = T1 K is never formed), the noised outputs
//            (the clean state before the tile: the fork), the clean outputs and the update.
//   waves 4 / 6 (G waves, clean / noised) prepare the next tile: K K^T with the k norms, the
//            decay/beta mask A, T by blocked forward substitution in fp32, the T1 and T2 operand
//            fragments.
//   waves 5 / 7 (P waves, clean / noised) prepare P with the q norms and decay folded in, and
//            own every row load of their stream: they store the next tile's v rows (v is
//            double-buffered) and the q and k rows of the tile after next, the latter into the
//            buffers of the current tile, once the state waves have read them (an LDS counter).
// The outputs of a tile are staged row-major in its spent v buffer and stored at the start of the
// next phase as 16-byte runs of whole rows (each state wave a quarter of the rows): a store
// instruction then covers four rows of 256 bytes, where a lane's own accumulator column gives two
// rows of 64 bytes per instruction (sixteen per stream; measured 574 vs 613 us at the 27B-class
// layer, 243 vs 252 us at the 0.8B-class one). The P waves refill that v buffer only after the
// same LDS counter, which the state waves raise after reading the staged rows.
// One barrier per tile; every operand the roles exchange is double-buffered by tile parity. Each
// SIMD runs one state wave beside one G or P wave.
// Sum of squares of row l32 of a [32 x 128] bf16 operand held as four rho-ordered fragments (lane
// (l32, h) holds 64 of the row's values): paired bf16 dot products into four fp32 partial sums,
// then the other half of the row from lane l32 + 32 (or l32 - 32), so both lanes get the row total.
__device__ __forceinline__ float row_sumsq(const Frag<true> (&f)[4]) {
  float s[4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    float x = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bf16x2 lo = {f[kt].lo[2 * i], f[kt].lo[2 * i + 1]};
      const bf16x2 hi = {f[kt].hi[2 * i], f[kt].hi[2 * i + 1]};
      x = __builtin_amdgcn_fdot2_f32_bf16(lo, lo, x, false);
      x = __builtin_amdgcn_fdot2_f32_bf16(hi, hi, x, false);
    }
    s[kt] = x;
  }
  const float half = (s[0] + s[1]) + (s[2] + s[3]);
  // the other half from lane l ^ 32 (LDS crossbar permute); the sum is commutative, so the two
  // lanes of a row hold bit-identical totals
  const float other = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((__lane_id() ^ 32) << 2,
                                                                            __builtin_bit_cast(int, half)));
  return half + other;
}

// Pipelined-kernel operand convention. The state S is held with its rows (d) permuted inside each
// 32-row slice: accumulator row rho(v, h) holds d = 16 h + v. Fed back as a B operand, value v of
// lane (n, h) then carries d = 16 h + v, so every A operand contracted with it (W, Q) is read as 16
// CONSECUTIVE d of its row: two 16-byte LDS reads instead of four 8-byte ones. Products whose two
// operands both come from LDS rows (K K^T, K Q^T) use the same reads for both: the contraction pairs
// equal d whatever the order.
__device__ __forceinline__ void lds_frag_c(const bf16* base, int h, Frag<true>& f) {
  const bf16* p = base + 16 * h;
  f.lo = *(const bf16x8*)p;
  f.hi = *(const bf16x8*)(p + 8);
}
// Transposed read (as lds_frag_tr) whose result lane r = 8 m + 4 h' + e receives column
// 16 h' + 4 m + e of the 32-column slice: an A operand whose product rows come out in the permuted
// d order above. The transpose read hands each group of four result lanes the four consecutive
// columns one source lane addresses, so only the column-group addresses change.
__device__ __forceinline__ void lds_frag_tr_d(const bf16* base, int row_stride, int lane, Frag<true>& f) {
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  const int s = lane & 15, j = s & 3;
  const bf16* p = base + (4 * (lane >> 5) + (s >> 2)) * row_stride + 16 * (j & 1) + 4 * (2 * ((lane >> 4) & 1) + (j >> 1));
  bf16x4 r[4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
    r[m] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p + 8 * m * row_stride));
  f.lo = __builtin_shufflevector(r[0], r[1], 0, 1, 2, 3, 4, 5, 6, 7);
  f.hi = __builtin_shufflevector(r[2], r[3], 0, 1, 2, 3, 4, 5, 6, 7);
}

struct PipeSmem {
  static constexpr int DK = 128;
  static constexpr int QROW = DK + 8;          // bf16 row stride of q, k, W and v rows
  static constexpr int FROW = 36;              // fp32 [32][32] scratch row stride
  static constexpr int ROWS = 32 * QROW * 2;   // one [32][QROW] bf16 buffer
  static constexpr int PB = 64 * 16 * 2;       // P operand fragment, lane-major
  static constexpr int T2B = 64 * 16 * 2;      // T2 operand fragment, lane-major
  static constexpr int VSB = 4 * 32 * 4;       // state-phase vectors: EGQ, RNK, EGLK, EG
  static constexpr int VAB = 4 * 32 * 4;       // G-wave vectors: GAML, BET, EG, EGL
  static constexpr int VPB = 2 * 32 * 4;       // P-wave vectors: GAML, EG
  static constexpr int FB = 32 * FROW * 4;
  static constexpr int YB = 16 * 20 * 4;
  // row buffers Q, K, V and operand fragments P, T1, T2, all [stream][parity]
  static constexpr int O_Q = 0;
  static constexpr int O_K = O_Q + 4 * ROWS;
  static constexpr int O_V = O_K + 4 * ROWS;
  static constexpr int O_P = O_V + 4 * ROWS;
  static constexpr int O_T1 = O_P + 4 * PB;
  static constexpr int O_T2 = O_T1 + 4 * T2B;
  static constexpr int O_VS = O_T2 + 4 * T2B;
  static constexpr int O_VA = O_VS + 4 * VSB;
  static constexpr int O_VP = O_VA + 2 * VAB;
  static constexpr int O_AF = O_VP + 2 * VPB;
  static constexpr int O_TF = O_AF + 2 * FB;
  static constexpr int O_YF = O_TF + 2 * FB;
  // v conv: per state wave, its 32 columns' weights [32][4] and bias [32] in fp32, and the carry:
  // the clean stream's last three raw v rows before the tile, [3][32] bf16
  static constexpr int CWB = 32 * 5 * 4;
  static constexpr int CRB = 3 * 32 * 2;
  // G-wave column factors per stream: beta_i / ||k_i|| and beta e^gamma / ||k|| (32 floats each)
  static constexpr int VGB = 2 * 32 * 4;
  static constexpr int O_VG = O_YF + 2 * YB;
  static constexpr int O_CW = O_VG + 2 * VGB;
  static constexpr int O_CR = O_CW + 4 * CWB;
  static constexpr int O_FLAG = O_CR + 4 * CRB;  // count of state waves done reading a tile's rows
  static constexpr int TOTAL = O_FLAG + 16;
  static_assert(TOTAL <= 160 * 1024, "LDS budget");
};
// vector slots (floats) inside the VS and VA blocks
enum { VS_EGQ = 0, VS_RNK = 32, VS_EGLK = 64, VS_EG = 96 };
enum { VA_GAML = 0, VA_BET = 32, VA_EG = 64, VA_EGL = 96 };
enum { VP_GAML = 0, VP_EG = 32 };
enum { VG_BR = 0, VG_C1 = 32 };

// Bit of the library's per-device status word (dllm_status): the bounded LDS row-buffer wait of
// the pipelined fork gave up (the launch's outputs are then invalid).
enum { STATUS_LDS_WAIT = 1u };
static __device__ unsigned dllm_status_word;

// One fp32 element of a state snapshot: a non-temporal store (nothing in the launch reads the
// snapshot back) at device scope, so that the line is written through to memory instead of held
// dirty in the XCD's L2 until the launch ends. Issued as its own instruction, which also keeps the
// compiler from moving the stores among the update's products. Measured at the 27B-class layer:
// the fork 559.6 vs 594.3 us with the compiler's non-temporal store (571.2 us for the same nt
// store issued this way, 562.3 us with system scope), bit-identical; 253.1 vs 259.2 us at the
// 0.8B-class layer.
// OFF: an immediate byte offset from p.
template <int OFF> __device__ __forceinline__ void store_snapshot(float* p, float v) {
  asm volatile("global_store_dword %0, %1, off offset:%2 nt sc1" ::"v"(p), "v"(v), "i"(OFF) : "memory");
}
// The 16 values of one 32-row slice of a state wave's accumulator: rows 32 kt + 16 h + v of the
// snapshot (p0 = row 32 kt + 16 h), 512 bytes apart, as immediate offsets from two base addresses
// (v < 8 and v >= 8) instead of an address formed per store. With the v conv on the state waves
// (whose VALU is then the bound) this measured 604 vs 611 us at the 27B-class fork and 260 vs
// 270 us at the 0.8B-class, bit-identical (before it: 581 vs 561 us, slower).
__device__ __forceinline__ void store_snapshot_slice(float* p0, const f32x16& s) {
  float* const p1 = p0 + 8 * 128;
  store_snapshot<0>(p0, s[0]);
  store_snapshot<512>(p0, s[1]);
  store_snapshot<1024>(p0, s[2]);
  store_snapshot<1536>(p0, s[3]);
  store_snapshot<2048>(p0, s[4]);
  store_snapshot<2560>(p0, s[5]);
  store_snapshot<3072>(p0, s[6]);
  store_snapshot<3584>(p0, s[7]);
  store_snapshot<0>(p1, s[8]);
  store_snapshot<512>(p1, s[9]);
  store_snapshot<1024>(p1, s[10]);
  store_snapshot<1536>(p1, s[11]);
  store_snapshot<2048>(p1, s[12]);
  store_snapshot<2560>(p1, s[13]);
  store_snapshot<3072>(p1, s[14]);
  store_snapshot<3584>(p1, s[15]);
}

__device__ __forceinline__ void report_status(unsigned bit) {
  __hip_atomic_fetch_or(&dllm_status_word, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// SPLIT: one workgroup per (sequence, value head, half of the value columns): state waves 0 and 1
// own columns [64 half + 32 u, +32) and state waves 2 and 3 only keep the barrier and counter
// sequence. The G and P waves prepare the whole tile in both workgroups of a head. For batches
// whose (sequence, head) count fills half the chip or less (measured: 302-306 vs 312-317 us at
// B = 8, Hv = 16, bit-identical).
// NS = 1: the same kernel over one stream (the chunked rule with per-chunk states, no fork): waves
// 6 and 7 keep the barrier sequence only, the state waves form the clean stream's products alone,
// and the state starts from a.init ([B, Hv, 128, 128] fp32) when it is given.
// VC (two streams; 1: bf16 conv weights, 2: fp32): the v rows are the short conv's inputs, and each
// state wave convolves its own columns of a tile's v rows in place (width 4, SiLU) before it reads
// them, in the conv kernel's arithmetic: the layer's conv then only writes the q and k channels.
template <bool SPLIT, int NS = 2, int VC = 0>
__global__ __launch_bounds__(512) void gdn_fork_pipe_kernel(GdnArgs a) {
  static_assert(VC == 0 || NS == 2, "the v conv runs with both streams");
  using SM = PipeSmem;
  using F = Frag<true>;
  constexpr int KT = 4;
  constexpr int QROW = SM::QROW, FROW = SM::FROW;
  constexpr float LOG2E = 1.4426950408889634f;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SM::TOTAL];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const bool prep = wave >= 4;
  const int u = wave & 3;            // state waves: column slice; prep waves: role
  const int gs = u >> 1;             // prep waves: stream prepared (0 clean, 1 noised)
  const bool isG = prep && (u & 1) == 0;

  const int lin = xcd_linear_id(blockIdx.x, gridDim.x);  // the halves of a head: one XCD
  const int half = SPLIT ? lin & 1 : 0;
  const int hv = (SPLIT ? lin >> 1 : lin) % a.Hv;
  const int b = (SPLIT ? lin >> 1 : lin) / a.Hv;
  const bool idle = SPLIT && !prep && u >= 2;
  const int cu = SPLIT ? half * 64 + (u & 1) * 32 : u * 32;  // first value column of a state wave
  const int hk = hv / (a.Hv / a.Hk);
  const int ntiles = a.T / a.sub;

  auto QB = [&](int s, int p) { return (bf16*)(smem + SM::O_Q + (2 * s + p) * SM::ROWS); };
  auto KB = [&](int s, int p) { return (bf16*)(smem + SM::O_K + (2 * s + p) * SM::ROWS); };
  auto T1f = [&](int s, int p) { return (bf16x8*)(smem + SM::O_T1 + (2 * s + p) * SM::T2B); };
  auto VB = [&](int s, int p) { return (bf16*)(smem + SM::O_V + (2 * s + p) * SM::ROWS); };
  auto PBf = [&](int s, int p) { return (bf16x8*)(smem + SM::O_P + (2 * s + p) * SM::PB); };
  auto T2f = [&](int s, int p) { return (bf16x8*)(smem + SM::O_T2 + (2 * s + p) * SM::T2B); };
  auto VS = [&](int s, int p) { return (float*)(smem + SM::O_VS + (2 * s + p) * SM::VSB); };
  auto VA = [&](int s) { return (float*)(smem + SM::O_VA + s * SM::VAB); };
  auto VP = [&](int s) { return (float*)(smem + SM::O_VP + s * SM::VPB); };
  unsigned* const flag = (unsigned*)(smem + SM::O_FLAG);
  auto AFf = [&](int s) { return (float*)(smem + SM::O_AF + s * SM::FB); };
  auto TFf = [&](int s) { return (float*)(smem + SM::O_TF + s * SM::FB); };
  auto YFf = [&](int s) { return (float*)(smem + SM::O_YF + s * SM::YB); };
  auto VGf = [&](int s) { return (float*)(smem + SM::O_VG + s * SM::VGB); };
  auto CWf = [&](int w) { return (float*)(smem + SM::O_CW + w * SM::CWB); };
  auto CRf = [&](int w) { return (bf16*)(smem + SM::O_CR + w * SM::CRB); };

  // ---- prep waves: loads. The P wave of each stream (wave 5 / 7) loads that stream's q, k and v
  // rows, so that the G waves, whose preparation chain is the longest, issue no row loads: lane
  // (row group lr0, segment lseg) holds columns [8 lseg, +8) of tile rows lr0 + 4 i, i = 0..7
  // (sixteen lanes per row: every load and LDS write instruction covers four whole 256-byte rows,
  // so the LDS writes are free of bank conflicts). The G waves load g and beta.
  const int lr0 = lane >> 4, lseg = lane & 15;
  const int e0 = lseg * 8;
  bf16x8 rq[8], rk[8], rv[8];
  float rg = 0.f, rb = 0.f, rgp = 0.f;
  auto issue_loads = [&](int tq, int tvv) {  // q/k (and g, beta) of tile tq, v of tile tvv; -1 = none
    if (prep && !isG) {
      const GdnStream& st = a.s[gs];
      const bf16* const qb = (const bf16*)st.q + b * a.q_sb + (long long)hk * a.q_sh + e0;
      const bf16* const kb = (const bf16*)st.k + b * a.k_sb + (long long)hk * a.k_sh + e0;
      const bf16* const vb = (const bf16*)st.v + b * a.v_sb + (long long)hv * a.v_sh + e0;
      // unconditional loads (a tile index of -1 reloads tile 0, unused), so that the compiler
      // counts them exactly and the load phase waits only for the row it writes
      const int tqq = tq < 0 ? 0 : tq, tvq = tvv < 0 ? 0 : tvv;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = lr0 + 4 * i;
        const int rr = r < a.sub ? r : 0;  // rows >= sub are zero padding (loaded from row 0, zeroed on use)
        rq[i] = *(const bf16x8*)(qb + (tqq * a.sub + rr) * a.q_st);
        rk[i] = *(const bf16x8*)(kb + (tqq * a.sub + rr) * a.k_st);
        rv[i] = *(const bf16x8*)(vb + (tvq * a.sub + rr) * a.v_st);
      }
      rgp = st.g[b * a.g_sb + (long long)hv * a.g_sh + (tqq * a.sub + min(l32, a.sub - 1)) * a.g_st];
    }
    // g and beta: every lane loads (padding rows from the last real row, zeroed on use), so that
    // no constant is ever written to these registers while a load into them may be in flight
    // (such a write makes the compiler wait for every outstanding load right after the issue)
    if (isG && tq >= 0) {
      const GdnStream& st = a.s[gs];
      const int row = tq * a.sub + min(l32, a.sub - 1);
      rg = st.g[b * a.g_sb + (long long)hv * a.g_sh + row * a.g_st];
      rb = st.beta[b * a.b_sb + (long long)hv * a.b_sh + row * a.b_st];
    }
  };

  // inclusive scan of g over the tile's rows (lanes 0..31 and, in `both`, 32..63 alike): the
  // cumulative decay gamma of row l32; rows >= sub contribute zero
  auto gamma_scan = [&](float g, bool both) {
    float x = ((both || h == 0) && l32 < a.sub) ? g : 0.f;
    x += dpp_mov<0x111>(x);  // row_shr:1
    x += dpp_mov<0x112>(x);  // row_shr:2
    x += dpp_mov<0x114>(x);  // row_shr:4
    x += dpp_mov<0x118>(x);  // row_shr:8
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x142, 0xA, 0xF, false));
    return x;
  };
  const bf16x8 vzero = {};
  // raw rows of one tile from this P wave's registers into LDS; rows >= sub are written as zeros
  // (whole tiles take the branch without selects)
  auto put_rows = [&](bf16* dst, const bf16x8* src) {
    dst += e0;
    if (a.sub == 32) {
#pragma unroll
      for (int i = 0; i < 8; ++i) *(bf16x8*)(dst + (lr0 + 4 * i) * QROW) = src[i];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = lr0 + 4 * i;
        *(bf16x8*)(dst + r * QROW) = r < a.sub ? src[i] : vzero;
      }
    }
  };

  // One barrier per tile. In the phase of tile c, the state waves run tile c; the G and P waves
  // prepare tile c + 1 from its rows, which are in LDS since the phase before; the P waves then
  // store tile c + 1's v rows (v is double-buffered) and, once every state wave has read tile c's
  // q and k rows (the LDS counter `flag`), tile c + 2's q and k rows into the buffers of tile c.
  // The roles run separate loops with the same barrier sequence, so that neither role's registers
  // (prefetched rows, the state) are held live through the other.
  if (tid == 0) {
    flag[0] = 0u;  // the P waves' row-buffer count
    flag[1] = 0u;  // column split with the v conv: tiles convolved for state waves 0 and 1
    flag[2] = 0u;
  }
  if constexpr (NS == 1) {
    if (prep && gs == 1) {  // no second stream: the barrier sequence of the prep loop only
      for (int c = -1; c < ntiles; ++c) __syncthreads();
      return;
    }
  }
  if (prep) {
  // the G waves carry the longest chain of a tile: the SIMD arbiter serves them first
  if (isG) __builtin_amdgcn_s_setprio(2);
  issue_loads(0, -1);
  if (!isG) {
    put_rows(QB(gs, 0), rq);
    put_rows(KB(gs, 0), rk);
  }
  for (int c = -1; c < ntiles; ++c) {
    const int lo = opaque_v(l32), ho = opaque_v(h);  // lane indices for masks (see opaque_v)
    __syncthreads();  // tile c-1's state phase and tile c's preparation are done
    if (c + 1 < ntiles) {
      // cumulative decay of tile c + 1 from the registers loaded in the phase before
      const int pn = (c + 1) & 1;
      if (isG) {
        const float gam = gamma_scan(rg, false);
        const float gall = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gam), 31));
        if (h == 0) {
          float* va = VA(gs);
          va[VA_GAML + l32] = gam * LOG2E;
          va[VA_BET + l32] = l32 < a.sub ? rb : 0.f;
          va[VA_EG + l32] = __builtin_amdgcn_exp2f(gam * LOG2E);
          va[VA_EGL + l32] = __builtin_amdgcn_exp2f((gall - gam) * LOG2E);
        }
      } else {
        const float gam = gamma_scan(rgp, false);
        if (h == 0) {
          float* vp = VP(gs);
          vp[VP_GAML + l32] = gam * LOG2E;
          vp[VP_EG + l32] = __builtin_amdgcn_exp2f(gam * LOG2E);
        }
      }
      wave_lds_sync();
      (void)pn;
    }
    if (c + 1 < ntiles) issue_loads(c + 2 < ntiles ? c + 2 : -1, c + 1);

    // ------------------------------------------------------------ preparation of tile c + 1
    {
      if (c + 1 < ntiles) {
        const int pn = (c + 1) & 1;
        const float* va = VA(gs);
        float* const vs = VS(gs, pn);
        const bf16* const K = KB(gs, pn);
        f32x4 gam4[4];
        if (isG) {
          // A = mask(beta_i k^_i . k^_j e^(gamma_i - gamma_j)), j < i, from the Gram K K^T
          float* const AF = AFf(gs);
          float* const TF = TFf(gs);
          float* const YF = YFf(gs);
          f32x16 acc = zero16();
          F fa[KT];
#pragma unroll
          for (int kt = 0; kt < KT; ++kt) lds_frag_c(K + l32 * QROW + kt * 32, h, fa[kt]);
#pragma unroll
          for (int m = 0; m < 4; ++m) gam4[m] = *(const f32x4*)(va + VA_GAML + 8 * m + 4 * h);
#pragma unroll
          for (int kt = 0; kt < KT; ++kt) mma32(acc, fa[kt], fa[kt]);
          __builtin_amdgcn_sched_group_barrier(0x100, 2 * KT + 4, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 2 * KT, 0);
          // k row norms from the Gram operands while the products run: lane (l32, h) holds half
          // of row l32; the row's 1/||k|| goes to the state vectors and comes back as row vectors
          const float rj = a.l2norm ? rsqrtf(row_sumsq(fa) + 1e-6f) : 1.f;
          const float eglj = va[VA_EGL + l32];
          float* const vg = VGf(gs);
          if (h == 0) {
            vs[VS_EGLK + l32] = eglj * rj;
            vs[VS_RNK + l32] = rj;
            vs[VS_EG + l32] = va[VA_EG + l32];
            // per-row factors of A and T1, formed once per row instead of once per element (the
            // same products in the same order)
            const float bet = va[VA_BET + l32];
            vg[VG_BR + l32] = bet * rj;
            vg[VG_C1 + l32] = bet * va[VA_EG + l32] * rj;
          }
          wave_lds_sync();
          const float gj = va[VA_GAML + l32];
          f32x4 br4[4];
#pragma unroll
          for (int m = 0; m < 4; ++m) br4[m] = *(const f32x4*)(vg + VG_BR + 8 * m + 4 * h);
#pragma unroll
          for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int i = 8 * m + 4 * h + e;
              const float val = (br4[m][e] * rj) * acc[4 * m + e] * __builtin_amdgcn_exp2f(gam4[m][e] - gj);
              AF[i * FROW + l32] = (lo < 8 * m + 4 * ho + e) ? val : 0.f;
            }
          wave_lds_sync();
          // level 0: four 8x8 diagonal blocks, one column per lane (lanes 0..31); lanes of odd
          // blocks also clear the block above (read as zero by level 2)
          if (h == 0) {
            const int bb = l32 >> 3, cc = lo & 7, o = 8 * bb;
            f32x4 ar[8][2];
#pragma unroll
            for (int i = 1; i < 8; ++i) {
              ar[i][0] = *(const f32x4*)(AF + (o + i) * FROW + o);
              ar[i][1] = *(const f32x4*)(AF + (o + i) * FROW + o + 4);
            }
            float x[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = (i == cc) ? 1.f : 0.f;
#pragma unroll
            for (int i = 1; i < 8; ++i) {
              float sacc = 0.f;
#pragma unroll
              for (int j = 0; j < i; ++j) sacc = __builtin_fmaf(ar[i][j >> 2][j & 3], x[j], sacc);
              if (i > cc) x[i] = -sacc;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) TF[(o + i) * FROW + o + cc] = x[i];
            if (bb & 1) {
#pragma unroll
              for (int i = 0; i < 8; ++i) TF[(o - 8 + i) * FROW + o + cc] = 0.f;
            }
          }
          wave_lds_sync();
          // level 1: T[m+1][m] = -D[m+1] (A[m+1][m] D[m]) for the sub-diagonal 8x8 blocks m = 0 and 2
          // (inside the 16x16 diagonal blocks; the block m = 1 lies in T[16:32][0:16], which level 2
          // writes whole without reading it)
          {
            const int ii = lane >> 3, jj = lane & 7;
            f32x4 arow[2][2];
            float dcol[2][8];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              const int m = 2 * q;
              arow[q][0] = *(const f32x4*)(AF + (8 * (m + 1) + ii) * FROW + 8 * m);
              arow[q][1] = *(const f32x4*)(AF + (8 * (m + 1) + ii) * FROW + 8 * m + 4);
#pragma unroll
              for (int kk = 0; kk < 8; ++kk) dcol[q][kk] = TF[(8 * m + kk) * FROW + 8 * m + jj];
            }
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              float sacc = 0.f;
#pragma unroll
              for (int kk = 0; kk < 8; ++kk) sacc = __builtin_fmaf(arow[q][kk >> 2][kk & 3], dcol[q][kk], sacc);
              YF[q * 64 + ii * 8 + jj] = sacc;
            }
            wave_lds_sync();
            f32x4 drow[2][2];
            float ycol[2][8];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              const int m = 2 * q;
              drow[q][0] = *(const f32x4*)(TF + (8 * (m + 1) + ii) * FROW + 8 * (m + 1));
              drow[q][1] = *(const f32x4*)(TF + (8 * (m + 1) + ii) * FROW + 8 * (m + 1) + 4);
#pragma unroll
              for (int kk = 0; kk < 8; ++kk) ycol[q][kk] = YF[q * 64 + kk * 8 + jj];
            }
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              const int m = 2 * q;
              float sacc = 0.f;
#pragma unroll
              for (int kk = 0; kk < 8; ++kk) sacc = __builtin_fmaf(drow[q][kk >> 2][kk & 3], ycol[q][kk], sacc);
              TF[(8 * (m + 1) + ii) * FROW + 8 * m + jj] = -sacc;
            }
          }
          wave_lds_sync();
          // level 2: T[16:32][0:16] = -T22 (A21 T11) as fp32 16x16x4 matrix products (lane l supplies
          // A[l % 16][l / 16] and B[l / 16][l % 16] and holds D[4 (l / 16) + v][l % 16]), the
          // intermediate through YF; on the VALU this level was 128 FMAs per lane, on a SIMD whose
          // VALU the state wave beside it needs (27B-class fork 623 vs 649 us; the outputs measured
          // bit-identical to the FMA form, whose sums ran in the same k order)
          {
            const int li = lane & 15, lk = lane >> 4;
            f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
              y = __builtin_amdgcn_mfma_f32_16x16x4f32(AF[(16 + li) * FROW + 4 * kb + lk], TF[(4 * kb + lk) * FROW + li], y,
                                                       0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) YF[(4 * lk + v) * 20 + li] = y[v];
            wave_lds_sync();
            f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
              z = __builtin_amdgcn_mfma_f32_16x16x4f32(TF[(16 + li) * FROW + 16 + 4 * kb + lk], YF[(4 * kb + lk) * 20 + li],
                                                       z, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) TF[(16 + 4 * lk + v) * FROW + li] = -z[v];
          }
          wave_lds_sync();
          // T1 = T diag(beta e^gamma / ||k||) and T2 = T diag(beta) as operand fragments
          // (lane = row l32, columns rho(v, h); lower triangle with the diagonal)
          f32x16 tv1, tv2;
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const f32x4 t4 = *(const f32x4*)(TF + l32 * FROW + 8 * m + 4 * h);
            const f32x4 be4 = *(const f32x4*)(va + VA_BET + 8 * m + 4 * h);
            const f32x4 c14 = *(const f32x4*)(vg + VG_C1 + 8 * m + 4 * h);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const bool in = 8 * m + 4 * ho + e <= lo;
              tv1[4 * m + e] = in ? -(t4[e] * c14[e]) : 0.f;  // -T1
              tv2[4 * m + e] = in ? t4[e] * be4[e] : 0.f;
            }
          }
          F f1, f2;
          acc_to_frag(tv1, f1);
          acc_to_frag(tv2, f2);
          bf16x8* t2d = T2f(gs, pn) + 2 * lane;
          t2d[0] = f2.lo;
          t2d[1] = f2.hi;
          // -T1 as the A operand of V' = U - T1 (K S): the state waves apply it to their K S
          bf16x8* t1d = T1f(gs, pn) + 2 * lane;
          t1d[0] = f1.lo;
          t1d[1] = f1.hi;
        } else {
          // P^T = K Q^T: lane = query row l32, values = key rows rho(v, h); P_ij = mask(scale/||q_i||
          // q_i . k^_j e^(gamma_i - gamma_j)), j <= i, with 1/||k_j|| applied to V' instead
          const bf16* const Q = QB(gs, pn);
          F fq[KT], fk[KT];
#pragma unroll
          for (int kt = 0; kt < KT; ++kt) {
            lds_frag_c(Q + l32 * QROW + kt * 32, h, fq[kt]);
            lds_frag_c(K + l32 * QROW + kt * 32, h, fk[kt]);
          }
#pragma unroll
          for (int m = 0; m < 4; ++m) gam4[m] = *(const f32x4*)(VP(gs) + VP_GAML + 8 * m + 4 * h);
          f32x16 acc = zero16();
#pragma unroll
          for (int kt = 0; kt < KT; ++kt) mma32(acc, fk[kt], fq[kt]);
          __builtin_amdgcn_sched_group_barrier(0x100, 4 * KT + 4, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 2 * KT, 0);
          const float gi = VP(gs)[VP_GAML + l32];
          // scale / ||q|| of query row l32 from this lane's half of the row and the other half's
          const float rqi = a.l2norm ? a.scale * rsqrtf(row_sumsq(fq) + 1e-6f) : a.scale;
          // P is kept as the A operand fragment of P V' (lane = query row, values = key rows in
          // rho order: the accumulator's own layout), lane-major
          f32x16 pv;
#pragma unroll
          for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float val = rqi * acc[4 * m + e] * __builtin_amdgcn_exp2f(gi - gam4[m][e]);
              pv[4 * m + e] = (8 * m + 4 * ho + e <= lo) ? val : 0.f;
            }
          F fpo;
          acc_to_frag(pv, fpo);
          bf16x8* const pd = PBf(gs, pn) + 2 * lane;
          pd[0] = fpo.lo;
          pd[1] = fpo.hi;
          if (h == 0) vs[VS_EGQ + l32] = VP(gs)[VP_EG + l32] * rqi;
        }
      }
    }
    if (!isG && c + 1 < ntiles) {
      // tile c + 1's v rows into the other v buffer and tile c + 2's q and k rows into tile c's
      // buffers, once every state wave has read tile c's q and k rows and the outputs of tile c - 1
      // staged in that v buffer (the state waves raise `flag` by one each per tile after both; the
      // wait is bounded, and they reach their raise without waiting on this wave)
      const unsigned target = 4u * (unsigned)(c + 1) + (unsigned)a.wait_bias;
      for (int spin = 0;; ++spin) {
        if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) break;
        if (spin >= a.spin_limit) {  // never expected: the state waves reach their raise unconditionally
          if (lane == 0) report_status(STATUS_LDS_WAIT);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      asm volatile("" ::: "memory");
      put_rows(VB(gs, (c + 1) & 1), rv);
      if (c + 2 < ntiles) {
        put_rows(QB(gs, c & 1), rq);
        put_rows(KB(gs, c & 1), rk);
      }
    }
  }
  } else {
  // ---- state waves: the clean state of value columns [32u, 32u + 32)
  f32x16 S[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) S[t] = zero16();
  if constexpr (NS == 1) {
    if (a.init) {  // an initial state [B, Hv, 128, 128] (rows as stored below)
      const float* ip = a.init + ((long long)b * a.Hv + hv) * (128LL * 128) + cu + 16 * h * 128 + l32;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) S[kt][v] = ip[(32 * kt + v) * 128];
    }
  }
  if (a.fork_init) {  // a range after the first block: the snapshot before it (rows as stored below)
    const float* ip = a.fork_init + ((long long)b * a.snap_rows * a.Hv + hv) * (128LL * 128) + cu + 16 * h * 128 + l32;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int v = 0; v < 16; ++v) S[kt][v] = ip[(32 * kt + v) * 128];
  }
  if constexpr (VC) {
    // this wave's conv weights and bias, and the carry before the first tile: the clean stream's
    // raw v rows t_first - 3 .. t_first - 1 of its columns (zero before the sequence start)
    if (!idle) {
      float* const cw = CWf(u);
      bf16* const cr = CRf(u);
      if (lane < 32) {
        const long long ch = (long long)hv * 128 + cu + lane;  // v channel
        float w4[4], bias = 0.f;
        if (VC == 2) {
          const float* wp = (const float*)a.vconv_w + ch * 4;
#pragma unroll
          for (int j = 0; j < 4; ++j) w4[j] = wp[j];
          if (a.vconv_b) bias = ((const float*)a.vconv_b)[ch];
        } else {
          const bf16* wp = (const bf16*)a.vconv_w + ch * 4;
#pragma unroll
          for (int j = 0; j < 4; ++j) w4[j] = (float)wp[j];
          if (a.vconv_b) bias = (float)((const bf16*)a.vconv_b)[ch];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) cw[4 * lane + j] = w4[j];
        cw[128 + lane] = bias;
      }
      const bf16* const vb = (const bf16*)a.s[0].v + b * a.v_sb + (long long)hv * a.v_sh + cu;
      for (int i = lane; i < 96; i += 64) {
        const int r = i >> 5, col = i & 31;
        cr[i] = a.t_first - 3 + r >= 0 ? vb[(r - 3) * a.v_st + col] : (bf16)0.f;
      }
    }
  }
  // VC: the conv of 32 columns [cv, cv + 32) of tile c's v rows, both streams, in place, with the
  // weights and carry of state-wave slot w (the slot that owns those columns). Lane (p, g) takes
  // columns cv + 2p, +1 of rows 8g .. 8g + 7; the three rows before the tile are the carry (every
  // tile is one block, and the noised block starts from the clean rows before it), which then moves
  // on to this tile's last three clean rows. Rows >= sub stay zero. vconv_read takes every raw value
  // this lane needs; other lanes overwrite some of them in vconv_write, so a compiler fence must
  // separate the two (LDS keeps one wave's accesses in order). Without the column split each state
  // wave convolves its own columns; with it, the state waves 2 and 3, which own no columns, convolve
  // those of waves 0 and 1 and raise a per-slot LDS counter that waves 0 and 1 wait for.
  unsigned xr[2][11], nc = 0;
  f32x4 wa, wb;
  float ba, bb;
  auto vconv_read = [&](int c, int pc, int cv, int w) {
    const int p = lane & 15, g = lane >> 4;
    const bf16* const cr = CRf(w);
    if (a.vtails && lane < 48) {
      // the carry is this block's conv tails: elements 2 lane, +1 of the wave's [32 channels][3]
      const int e0 = 2 * lane, e1 = e0 + 1;
      const unsigned t0 = __builtin_bit_cast(unsigned short, cr[32 * (e0 % 3) + e0 / 3]);
      const unsigned t1 = __builtin_bit_cast(unsigned short, cr[32 * (e1 % 3) + e1 / 3]);
      const long long row = (long long)b * a.snap_rows + a.t_first / a.sub + c;
      *(unsigned*)((bf16*)a.vtails + (row * a.tails_cd + hv * 128 + cv) * 3 + e0) = t0 | (t1 << 16);
    }
    const float* const cw = CWf(w);
    wa = *(const f32x4*)(cw + 8 * p);
    wb = *(const f32x4*)(cw + 8 * p + 4);
    ba = cw[128 + 2 * p];
    bb = cw[129 + 2 * p];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const bf16* const vb = VB(s, pc) + cv + 2 * p;
#pragma unroll
      for (int i = 0; i < 3; ++i)
        xr[s][i] = *(const unsigned*)(g == 0 ? cr + 32 * i + 2 * p : vb + (8 * g - 3 + i) * QROW);
#pragma unroll
      for (int i = 3; i < 11; ++i) xr[s][i] = *(const unsigned*)(vb + (8 * g + i - 3) * QROW);
    }
    if (g < 3) {
      const int q = a.sub - 3 + g;  // the carry's row g for the next tile
      nc = *(const unsigned*)(q >= 0 ? VB(0, pc) + cv + 2 * p + q * QROW : cr + 32 * (q + 3) + 2 * p);
    }
  };
  // the two columns' values rounded to bf16 together (one packed conversion), as a bf16 pair
  auto pack_bf16 = [](float x0, float x1) -> unsigned {
    const f32x2 v = {x0, x1};
    return __builtin_bit_cast(unsigned, __builtin_convertvector(v, bf16x2));
  };
  auto vconv_write = [&](int pc, int cv, int w) {
    const int p = lane & 15, g = lane >> 4;
    unsigned out[2][8];
    // per stream: the sums, then the SiLU (silu_f32's steps) in stages over all 16 values, so that
    // the exponentials and reciprocals of different values follow each other instead of each
    // waiting on its own (no hazard wait states; 0.8B-class fork 282 vs 285 us, bit-identical)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float a0[8], a1[8], e0[8], e1[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        float acc0 = ba, acc1 = bb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const unsigned x = xr[s][r + j];
          acc0 = __builtin_fmaf(wa[j], __builtin_bit_cast(float, x << 16), acc0);
          acc1 = __builtin_fmaf(wb[j], __builtin_bit_cast(float, x & 0xffff0000u), acc1);
        }
        if (VC == 1) {  // bf16 weights: the sum is rounded to bf16 before the SiLU
          const unsigned rr = pack_bf16(acc0, acc1);
          acc0 = __builtin_bit_cast(float, rr << 16);
          acc1 = __builtin_bit_cast(float, rr & 0xffff0000u);
        }
        a0[r] = acc0;
        a1[r] = acc1;
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        e0[r] = __builtin_amdgcn_exp2f(-1.4426950408889634f * a0[r]);
        e1[r] = __builtin_amdgcn_exp2f(-1.4426950408889634f * a1[r]);
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        e0[r] = __builtin_amdgcn_rcpf(1.0f + e0[r]);
        e1[r] = __builtin_amdgcn_rcpf(1.0f + e1[r]);
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) out[s][r] = pack_bf16(a0[r] * e0[r], a1[r] * e1[r]);
    }
    if (a.sub < 32) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int r = 0; r < 8; ++r)
          if (8 * g + r >= a.sub) out[s][r] = 0u;
    }
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int r = 0; r < 8; ++r) *(unsigned*)(VB(s, pc) + cv + 2 * p + (8 * g + r) * QROW) = out[s][r];
    if (g < 3) *(unsigned*)(CRf(w) + 32 * g + 2 * p) = nc;
  };
  auto vconv = [&](int c, int pc, int cv, int w) {
    vconv_read(c, pc, cv, w);
    asm volatile("" ::: "memory");  // every raw value read before any lane writes its outputs
    vconv_write(pc, cv, w);
  };
  for (int c = -1; c < ntiles; ++c) {
    __syncthreads();  // tile c-1's state phase and tile c's preparation are done
    if (idle) {  // the other half's columns: count as done reading the tile's rows
      if (c >= 0 && lane == 0) __hip_atomic_fetch_add(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if constexpr (VC != 0) {
        if (c >= 0) {
          // the conv of state wave (u & 1)'s columns, then its counter (after the LDS writes land)
          const int w = u & 1;
          vconv(c, c & 1, half * 64 + w * 32, w);
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          if (lane == 0) __hip_atomic_fetch_add(flag + 1 + w, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
      }
      continue;
    }
    if (c >= 0) {
      // ---------------------------------------------------------- state phase, tile c
      const int pc = c & 1;
      const int t0 = c * a.sub;
      const int rs = opaque(a.Hv * a.Dv);  // token stride of the outputs
      if (c >= 1) {
        // tile c - 1's outputs, staged row-major in its spent v buffers by every state wave, go out
        // as 16-byte runs of whole rows: this wave's share of the rows, with the workgroup's
        // columns (all 128, or the 64 of its half of the head)
        constexpr int NCOL = SPLIT ? 64 : 128, NACT = SPLIT ? 2 : 4;
        constexpr int LPR = NCOL / 8, RPI = 64 / LPR, RPW = 32 / NACT;  // lanes per row, rows per store, rows per wave
        const int col0 = SPLIT ? 64 * half : 0;
        const int rr = lane / LPR, ch = lane % LPR;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const bf16* const st = VB(s, pc ^ 1);
          bf16* const ob = (bf16*)a.s[s].out + ((long long)b * a.t_rows + t0 - a.sub) * rs + (long long)hv * a.Dv + col0 + 8 * ch;
#pragma unroll
          for (int i = 0; i < RPW / RPI; ++i) {
            const int row = u * RPW + i * RPI + rr;
            const bf16x8 o8 = *(const bf16x8*)(st + row * QROW + col0 + 8 * ch);
            if (row < a.sub) *(bf16x8*)(ob + (long long)row * rs) = o8;
          }
        }
      }
      // K S and Q S of both streams from the clean state before the tile; the K and Q fragments
      // of slice kt + 1 are read while the products of slice kt run
      if constexpr (VC != 0 && !SPLIT) {
        vconv(c, pc, cu, u);
        __builtin_amdgcn_sched_barrier(0);
      }
      f32x16 accKS[NS], accQS[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        accKS[s] = zero16();
        accQS[s] = zero16();
      }
      F fk2[2][NS], fq[2][NS];  // [slice parity][stream]
      auto read_kq = [&](int kt) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          lds_frag_c(KB(s, pc) + l32 * QROW + kt * 32, h, fk2[kt & 1][s]);
          lds_frag_c(QB(s, pc) + l32 * QROW + kt * 32, h, fq[kt & 1][s]);
        }
      };
      read_kq(0);
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        F sx;
        acc_to_frag(S[kt], sx);
        if (kt + 1 < KT) read_kq(kt + 1);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          mma32(accKS[s], fk2[kt & 1][s], sx);
          mma32(accQS[s], fq[kt & 1][s], sx);
        }
      }
      // issue order: slice 0's reads, then each slice's products behind the next slice's reads
      // (keeps eight LDS reads in flight per wave)
      __builtin_amdgcn_sched_group_barrier(0x100, 4 * NS, 1);
#pragma unroll
      for (int kt = 0; kt + 1 < KT; ++kt) {
        __builtin_amdgcn_sched_group_barrier(0x100, 4 * NS, 1);
        __builtin_amdgcn_sched_group_barrier(0x008, 4 * NS, 1);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4 * NS, 1);
      // the clean k rows as the A operand of the state update, read now: after them this wave has
      // read every q and k row of tile c, and the P waves may overwrite those buffers
      F fku[KT];
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) lds_frag_tr_d(KB(0, pc) + kt * 32, QROW, lane, fku[kt]);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane == 0) __hip_atomic_fetch_add(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if constexpr (VC != 0 && SPLIT) {
        // this wave's columns of the v rows are convolved by state wave u + 2: wait for its count
        // (bounded; it never waits on this wave inside a phase)
        const unsigned target = (unsigned)(c + 1) + (unsigned)a.wait_bias;
        for (int spin = 0;; ++spin) {
          if (__hip_atomic_load(flag + 1 + u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) break;
          if (spin >= a.spin_limit) {
            if (lane == 0) report_status(STATUS_LDS_WAIT);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
        asm volatile("" ::: "memory");
      }
      // V' = U - T1 (K S) = T2 V + (-T1) (K S): W = T1 K is never formed; K S feeds straight back
      // as the B operand of the -T1 product (its rows are the tile rows in rho order)
      f32x16 accV[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        accV[s] = zero16();
        F ft, fv, ft1, fks;
        const bf16x8* t2 = T2f(s, pc) + 2 * lane;
        ft.lo = t2[0];
        ft.hi = t2[1];
        const bf16x8* t1 = T1f(s, pc) + 2 * lane;
        ft1.lo = t1[0];
        ft1.hi = t1[1];
        lds_frag_tr(VB(s, pc) + cu, QROW, lane, fv);
        acc_to_frag(accKS[s], fks);
        mma32(accV[s], ft, fv);    // U = T2 V
        mma32(accV[s], ft1, fks);  // - T1 K S
      }
#pragma unroll
      for (int si = 0; si < NS; ++si) {
        const int s = NS - 1 - si;  // noised first: the clean update below overwrites S
        const float* vs = VS(s, pc);
        // O = diag(e^gamma scale/||q||) Q S + P (V' / ||k||),  V' = U - T1 K S
        f32x16 vn, vk;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const f32x4 egq = *(const f32x4*)(vs + VS_EGQ + 8 * m + 4 * h);
          const f32x4 rnk = *(const f32x4*)(vs + VS_RNK + 8 * m + 4 * h);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int v = 4 * m + e;
            vn[v] = accV[s][v];
            vk[v] = vn[v] * rnk[e];
            accQS[s][v] *= egq[e];
          }
        }
        {
          F fv, fp;
          acc_to_frag(vk, fv);
          const bf16x8* const pp = PBf(s, pc) + 2 * lane;
          fp.lo = pp[0];
          fp.hi = pp[1];
          mma32(accQS[s], fp, fv);
        }
        if (c + 1 < ntiles) {
          // staged row-major in this tile's v buffer (its v rows are spent: every state wave read
          // its own columns of them for U = T2 V above, and writes only those columns here), for
          // the 16-byte stores at the start of the next phase; rows >= sub are staged but not stored
          bf16* const st = VB(s, pc) + cu + l32 + 4 * h * QROW;
#pragma unroll
          for (int v = 0; v < 16; v += 2) {  // two values per conversion; rows rho(v), rho(v + 1)
            const unsigned pr = pack_bf16(accQS[s][v], accQS[s][v + 1]);
            *(unsigned short*)(st + (((v >> 2) << 3) + (v & 3)) * QROW) = (unsigned short)pr;
            *(unsigned short*)(st + ((((v + 1) >> 2) << 3) + ((v + 1) & 3)) * QROW) = (unsigned short)(pr >> 16);
          }
        } else {
          // the last tile of the launch: straight to the outputs
          bf16* ob = (bf16*)a.s[s].out + ((long long)b * a.t_rows + t0) * rs + (long long)hv * a.Dv + cu;
          const unsigned lo2 = (unsigned)(4 * h * rs + l32);
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int ru = ((v >> 2) << 3) + (v & 3);  // row = ru + 4h
            if (ru + 4 * h < a.sub) (ob + ru * rs)[lo2] = (bf16)accQS[s][v];
          }
        }
        if (s == 0) {
          // S <- e^gamma_last S + K_raw^T (e^(gamma_last - gamma) / ||k|| V'), snapshot after the tile
          const float lam = vs[VS_EG + 31];
          f32x16 vd;
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const f32x4 eglk = *(const f32x4*)(vs + VS_EGLK + 8 * m + 4 * h);
#pragma unroll
            for (int e = 0; e < 4; ++e) vd[4 * m + e] = vn[4 * m + e] * eglk[e];
          }
          F fd;
          acc_to_frag(vd, fd);
          // accumulator row rho(v, h) of slice kt is state row 32 kt + 16 h + v
          float* const sb = a.states ? a.states + (((long long)b * a.snap_rows + c) * a.Hv + hv) * (128LL * 128) + cu +
                                           16 * h * 128 + l32
                                     : nullptr;
#pragma unroll
          for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
            for (int v = 0; v < 16; ++v) S[kt][v] *= lam;
            mma32(S[kt], fku[kt], fd);
            if (sb) store_snapshot_slice(sb + 32 * kt * 128, S[kt]);
          }
        }
      }
    }
  }
  }
}

template <int DK, int DVW, bool BF16, bool FORK>
static int launch_gdn(const GdnArgs& a, hipStream_t st) {
  const int nwin = (a.Dv + DVW - 1) / DVW;
  const long long nblk = (long long)a.B * a.Hv * nwin;
  if (nblk > 0x7fffffff) return fail(DLLM_EUNSUPPORTED, "gdn: grid too large");
  gdn_chunk_kernel<DK, DVW, BF16, FORK><<<dim3((unsigned)nblk), dim3(FORK ? 512 : 256), 0, st>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "gdn launch: %s", hipGetErrorString(e));
  return DLLM_OK;
}

// Compute units of the current device (cached per device; 0 if the query fails).
static int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// 0: split a head's columns over two workgroups when the split grid fits the chip; 1: never;
// 2: always (dllm_set_fork_split, for tests)
static std::atomic<int> g_fork_split{0};

template <int NS, int VC = 0>
static int launch_fork_pipe(const GdnArgs& a, hipStream_t st) {
  const long long heads = (long long)a.B * a.Hv;
  const int mode = g_fork_split.load(std::memory_order_relaxed);
  const bool split = mode == 2 || (mode == 0 && 2 * heads <= device_cus());
  const long long nblk = split ? 2 * heads : heads;
  if (nblk > 0x7fffffff) return fail(DLLM_EUNSUPPORTED, "gdn: grid too large");
  if (split) gdn_fork_pipe_kernel<true, NS, VC><<<dim3((unsigned)nblk), dim3(512), 0, st>>>(a);
  else gdn_fork_pipe_kernel<false, NS, VC><<<dim3((unsigned)nblk), dim3(512), 0, st>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "gdn fork launch: %s", hipGetErrorString(e));
  return DLLM_OK;
}

static int gcd_int(int x, int y) {
  while (y) {
    int t = x % y;
    x = y;
    y = t;
  }
  return x;
}

// Column window per workgroup: bf16 covers the whole value head (up to 128 columns, one workgroup
// per (b, head)); fp32 operands take twice the LDS, so fp32 uses 64-column windows.
static int window_for(int dtype) { return dtype == DT_BF16 ? 128 : 64; }

static int dispatch_gdn(GdnArgs& a, int dtype, bool fork, hipStream_t st) {
  if (a.Dk > 128) return fail(DLLM_EUNSUPPORTED, "gdn: Dk=%d > 128 not supported", a.Dk);
  if (a.Dv > 128) return fail(DLLM_EUNSUPPORTED, "gdn: Dv=%d > 128 not supported", a.Dv);
  const int dk = a.Dk <= 64 ? 64 : 128;
  if (dtype == DT_BF16) {
    if (dk == 64) return fork ? launch_gdn<64, 128, true, true>(a, st) : launch_gdn<64, 128, true, false>(a, st);
    if (fork) return launch_gdn<128, 128, true, true>(a, st);
    // few (sequence, head) pairs (a decoding step: B = 1): two 64-column windows per head, so that
    // twice the workgroups share the state loads (the columns are independent)
    if ((long long)a.B * a.Hv < 128) return launch_gdn<128, 64, true, false>(a, st);
    return launch_gdn<128, 128, true, false>(a, st);
  }
  if (dtype == DT_F32) {
    if (dk == 64) return fork ? launch_gdn<64, 64, false, true>(a, st) : launch_gdn<64, 64, false, false>(a, st);
    if (fork) return fail(DLLM_EUNSUPPORTED, "gdn: fused fork needs Dk<=64 in fp32 (use the two-pass fork)");
    return launch_gdn<128, 64, false, false>(a, st);
  }
  return fail(DLLM_EUNSUPPORTED, "gdn: dtype %d not supported", dtype);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Sleeps after which a bounded wait gives up and sets a dllm_status bit (process-wide; tests lower
// it to force that path).
static std::atomic<int> g_spin_limit{1 << 20};
static std::atomic<int> g_wait_bias{0};  // dllm_set_wait_test_mode

static bool fits_i32(long long x) { return x >= -2147483647LL && x <= 2147483647LL; }

}  // namespace dllm

using namespace dllm;

extern "C" int dllm_gdn_fused_fork_supported(int Dk, int block, int dtype) {
  if (block <= 0 || 32 % block != 0) return 0;
  if (Dk <= 0 || Dk > 128) return 0;
  if (dtype == DT_F32 && Dk > 64) return 0;
  return dtype == DT_F32 || dtype == DT_BF16;
}

extern "C" int dllm_gdn_state_fork_path(int Dk, int Dv, int block, int dtype) {
  if (!dllm_gdn_fused_fork_supported(Dk, block, dtype)) return 0;
  return (dtype == DT_BF16 && Dk == 128 && Dv == 128) ? 2 : 1;
}

extern "C" int dllm_gdn_chunk_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                                  const void* v, const int64_t* v_strides, const float* g, const int64_t* g_strides,
                                  const float* beta, const int64_t* beta_strides, const float* initial_state,
                                  void* out, float* states, int B, int T, int Hk, int Hv, int Dk, int Dv,
                                  int chunk, int dtype, int use_qk_l2norm, float scale, void* stream) {
  if (!q || !k || !v || !g || !beta || !out || !q_strides || !k_strides || !v_strides || !g_strides || !beta_strides)
    return fail(DLLM_EINVAL, "gdn: null pointer");
  if (B <= 0 || T <= 0 || Hk <= 0 || Hv <= 0 || Dk <= 0 || Dv <= 0 || chunk <= 0)
    return fail(DLLM_EINVAL, "gdn: bad sizes B=%d T=%d Hk=%d Hv=%d Dk=%d Dv=%d chunk=%d", B, T, Hk, Hv, Dk, Dv, chunk);
  if (T % chunk) return fail(DLLM_EINVAL, "sequence_length %d is not a multiple of chunk_size %d", T, chunk);
  if (Hv % Hk) return fail(DLLM_EINVAL, "gdn: Hv=%d is not a multiple of Hk=%d", Hv, Hk);
  const int64_t* sts[5] = {q_strides, k_strides, v_strides, beta_strides, g_strides};
  const int H[5] = {Hk, Hk, Hv, Hv, Hv};
  for (int i = 0; i < 5; ++i)
    if (!fits_i32((long long)T * sts[i][1]) || !fits_i32((long long)H[i] * sts[i][2]) ||
        !fits_i32((long long)T * sts[i][1] + (long long)H[i] * sts[i][2]))
      return fail(DLLM_EUNSUPPORTED, "gdn: per-sequence extent exceeds 32-bit element offsets");
  GdnArgs a = {};
  GdnStream& s = a.s[0];
  s.q = q; s.k = k; s.v = v; s.g = g; s.beta = beta; s.out = out;
  a.q_sb = q_strides[0]; a.q_st = (int)q_strides[1]; a.q_sh = (int)q_strides[2];
  a.k_sb = k_strides[0]; a.k_st = (int)k_strides[1]; a.k_sh = (int)k_strides[2];
  a.v_sb = v_strides[0]; a.v_st = (int)v_strides[1]; a.v_sh = (int)v_strides[2];
  a.g_sb = g_strides[0]; a.g_st = (int)g_strides[1]; a.g_sh = (int)g_strides[2];
  a.b_sb = beta_strides[0]; a.b_st = (int)beta_strides[1]; a.b_sh = (int)beta_strides[2];
  a.s[1] = a.s[0];
  a.init = initial_state;
  a.states = states;
  a.B = B; a.T = T; a.Hk = Hk; a.Hv = Hv; a.Dk = Dk; a.Dv = Dv;
  a.sub = gcd_int(chunk, 32);
  a.snap_every = chunk / a.sub;
  a.scale = scale;
  a.l2norm = use_qk_l2norm;
  a.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  a.wait_bias = g_wait_bias.load(std::memory_order_relaxed);
  const int esz = dtype == DT_BF16 ? 2 : 4;
  const int vel = 16 / esz;
  auto st_ok = [&](const int64_t* st3) { return (st3[0] % vel == 0) && (st3[1] % vel == 0) && (st3[2] % vel == 0); };
  const int dkw = Dk <= 64 ? 64 : 128;
  a.vec_qk = aligned16(q) && aligned16(k) && st_ok(q_strides) && st_ok(k_strides) && Dk == dkw;
  a.vec_v = aligned16(v) && st_ok(v_strides) && (Dv % window_for(dtype) == 0);
  // bf16 heads of 128 x 128 with 16-byte rows and chunks that divide the 32-row tile: the pipelined
  // kernel on one stream, which prepares tile c + 1 beside the state work of tile c (measured at the
  // 27B-class clean pass 458 vs 758 us with the chunk kernel; 20 vs 20 us for one 32-token tile)
  if (dtype == DT_BF16 && Dk == 128 && Dv == 128 && a.vec_qk && a.vec_v && a.snap_every == 1) {
    a.t_rows = T;
    a.snap_rows = T / a.sub;
    a.fork_init = nullptr;
    return launch_fork_pipe<1>(a, (hipStream_t)stream);
  }
  return dispatch_gdn(a, dtype, false, (hipStream_t)stream);
}

// The state fork over blocks [kb0, kb1) of every sequence (the whole sequence: [0, L / block)).
// A range after the first block starts from states[:, kb0 - 1] and runs the pipelined kernel only.
// VConv (optional): the v channels come unconvolved from raw0 / rawt (same strides as qkv) and the
// kernel applies the width-4 conv + SiLU to them (weights [conv_dim, 4] of dtype_w, bias or null).
struct VConv {
  const void* raw0;
  const void* rawt;
  const void* weight;
  const void* bias;
  int dtype_w;
  void* tails;  // [B * nb, conv_dim, 3] (the v channels are written) or null
  int conv_dim;
};

static int state_fork(const void* qkv0, const void* qkvt, int64_t qkv_stride_b, int64_t qkv_stride_t,
                      const float* beta0, const float* betat, const float* g0, const float* gt, void* out0,
                      void* outt, float* states, int B, int L, int Hk, int Hv, int Dk, int Dv, int block, int dtype,
                      float scale, int kb0, int kb1, void* stream, const VConv* vc = nullptr) {
  if (!qkv0 || !qkvt || !beta0 || !betat || !g0 || !gt || !out0 || !outt) return fail(DLLM_EINVAL, "gdn fork: null pointer");
  if (vc) {
    if (!vc->raw0 || !vc->rawt || !vc->weight) return fail(DLLM_EINVAL, "gdn fork v conv: null pointer");
    if (vc->dtype_w != DT_BF16 && vc->dtype_w != DT_F32)
      return fail(DLLM_EUNSUPPORTED, "gdn fork v conv: weight dtype %d (bf16 or fp32)", vc->dtype_w);
    if (!(dtype == DT_BF16 && Dk == 128 && Dv == 128))
      return fail(DLLM_EUNSUPPORTED, "gdn fork v conv: needs the pipelined kernel (bf16, Dk = Dv = 128)");
  }
  if (B <= 0 || L <= 0 || Hk <= 0 || Hv <= 0 || Dk <= 0 || Dv <= 0 || block <= 0)
    return fail(DLLM_EINVAL, "gdn fork: bad sizes");
  if (L % block) return fail(DLLM_EINVAL, "L=%d is not a multiple of block=%d", L, block);
  if (Hv % Hk) return fail(DLLM_EINVAL, "gdn fork: Hv=%d is not a multiple of Hk=%d", Hv, Hk);
  if (!dllm_gdn_fused_fork_supported(Dk, block, dtype))
    return fail(DLLM_EUNSUPPORTED, "gdn fork: fused fork unsupported for Dk=%d block=%d dtype=%d", Dk, block, dtype);
  if (!fits_i32((long long)L * qkv_stride_t) || !fits_i32((long long)L * Hv))
    return fail(DLLM_EUNSUPPORTED, "gdn fork: per-sequence extent exceeds 32-bit element offsets");
  const int nb = L / block;
  if (kb0 < 0 || kb1 > nb || kb0 >= kb1) return fail(DLLM_EINVAL, "gdn fork: block range [%d, %d) of %d", kb0, kb1, nb);
  const bool whole = kb0 == 0 && kb1 == nb;
  if (kb0 > 0 && !states) return fail(DLLM_EINVAL, "gdn fork: a range after block 0 starts from states (null)");
  GdnArgs a = {};
  const int esz = dtype == DT_BF16 ? 2 : 4;
  const long long t_off = (long long)kb0 * block;  // first row of the range
  const char* base[2] = {(const char*)qkv0 + t_off * qkv_stride_t * esz, (const char*)qkvt + t_off * qkv_stride_t * esz};
  const char* vbase[2] = {base[0], base[1]};
  if (vc) {
    vbase[0] = (const char*)vc->raw0 + t_off * qkv_stride_t * esz;
    vbase[1] = (const char*)vc->rawt + t_off * qkv_stride_t * esz;
  }
  const float* bet[2] = {beta0 + t_off * Hv, betat + t_off * Hv};
  const float* gg[2] = {g0 + t_off * Hv, gt + t_off * Hv};
  void* outs[2] = {(char*)out0 + t_off * Hv * Dv * esz, (char*)outt + t_off * Hv * Dv * esz};
  for (int i = 0; i < 2; ++i) {
    GdnStream& s = a.s[i];
    s.q = base[i];
    s.k = base[i] + (long long)Hk * Dk * esz;
    s.v = vbase[i] + 2LL * Hk * Dk * esz;
    s.beta = bet[i];
    s.g = gg[i];
    s.out = outs[i];
  }
  a.q_sb = a.k_sb = a.v_sb = qkv_stride_b;
  a.q_st = a.k_st = a.v_st = (int)qkv_stride_t;
  a.q_sh = a.k_sh = Dk;
  a.v_sh = Dv;
  a.b_sb = a.g_sb = (long long)L * Hv;
  a.b_st = a.g_st = Hv;
  a.b_sh = a.g_sh = 1;
  a.init = nullptr;
  const long long snap_elems = (long long)Hv * Dk * Dv;
  a.states = states ? states + kb0 * snap_elems : nullptr;
  a.fork_init = kb0 > 0 ? states + (kb0 - 1) * snap_elems : nullptr;
  a.t_rows = L;
  a.snap_rows = nb;
  a.B = B; a.T = (kb1 - kb0) * block; a.Hk = Hk; a.Hv = Hv; a.Dk = Dk; a.Dv = Dv;
  a.sub = block;
  a.snap_every = 1;
  a.scale = scale;
  a.l2norm = 1;
  a.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  a.wait_bias = g_wait_bias.load(std::memory_order_relaxed);
  const int vel = 16 / esz;
  const bool st_ok = (qkv_stride_b % vel == 0) && (qkv_stride_t % vel == 0) && (Dk % vel == 0) && (Dv % vel == 0) &&
                     ((long long)Hk * Dk % vel == 0);
  const int dkw = Dk <= 64 ? 64 : 128;
  a.vec_qk = aligned16(qkv0) && aligned16(qkvt) && st_ok && Dk == dkw;
  a.vec_v = aligned16(vbase[0]) && aligned16(vbase[1]) && st_ok && (Dv % window_for(dtype) == 0);
  a.t_first = (int)t_off;
  if (vc) {
    if (!(a.vec_qk && a.vec_v))
      return fail(DLLM_EUNSUPPORTED, "gdn fork v conv: needs 16-byte aligned rows and strides");
    const long long wrow = 2LL * Hk * Dk;  // the first v channel's weight row
    const int wsz = vc->dtype_w == DT_F32 ? 4 : 2;
    a.vconv_w = (const char*)vc->weight + wrow * 4 * wsz;
    a.vconv_b = vc->bias ? (const char*)vc->bias + wrow * wsz : nullptr;
    if (vc->tails) {
      if ((uintptr_t)vc->tails % 4 || vc->conv_dim % 2 || vc->conv_dim < wrow + (long long)Hv * Dv)
        return fail(DLLM_EINVAL, "gdn fork v conv: tails need 4-byte alignment and an even conv_dim >= %lld",
                    wrow + (long long)Hv * Dv);
      a.vtails = (char*)vc->tails + wrow * 3 * esz;
      a.tails_cd = vc->conv_dim;
    }
    return vc->dtype_w == DT_F32 ? launch_fork_pipe<2, 2>(a, (hipStream_t)stream)
                                 : launch_fork_pipe<2, 1>(a, (hipStream_t)stream);
  }
  // full 128 x 128 heads with 16-byte rows: the pipelined kernel
  if (dtype == DT_BF16 && Dk == 128 && Dv == 128 && a.vec_qk && a.vec_v) return launch_fork_pipe<2>(a, (hipStream_t)stream);
  if (!whole) return fail(DLLM_EUNSUPPORTED, "gdn fork: block ranges need the pipelined kernel (bf16, Dk = Dv = 128)");
  return dispatch_gdn(a, dtype, true, (hipStream_t)stream);
}

extern "C" int dllm_gdn_state_fork_fwd(const void* qkv0, const void* qkvt, int64_t qkv_stride_b, int64_t qkv_stride_t,
                                       const float* beta0, const float* betat, const float* g0, const float* gt,
                                       void* out0, void* outt, float* states, int B, int L, int Hk, int Hv, int Dk,
                                       int Dv, int block, int dtype, float scale, void* stream) {
  const int nb = block > 0 && L > 0 && L % block == 0 ? L / block : 1;  // sizes are checked by state_fork
  return state_fork(qkv0, qkvt, qkv_stride_b, qkv_stride_t, beta0, betat, g0, gt, out0, outt, states, B, L, Hk, Hv,
                    Dk, Dv, block, dtype, scale, 0, nb, stream);
}

extern "C" int dllm_gdn_state_fork_range_fwd(const void* qkv0, const void* qkvt, int64_t qkv_stride_b,
                                             int64_t qkv_stride_t, const float* beta0, const float* betat,
                                             const float* g0, const float* gt, void* out0, void* outt, float* states,
                                             int B, int L, int Hk, int Hv, int Dk, int Dv, int block, int dtype,
                                             float scale, int block_begin, int block_end, void* stream) {
  return state_fork(qkv0, qkvt, qkv_stride_b, qkv_stride_t, beta0, betat, g0, gt, out0, outt, states, B, L, Hk, Hv,
                    Dk, Dv, block, dtype, scale, block_begin, block_end, stream);
}

extern "C" int dllm_gdn_state_fork_vconv_range_fwd(const void* qk0, const void* qkt, const void* raw0,
                                                   const void* rawt, int64_t stride_b, int64_t stride_t,
                                                   const void* conv_weight, const void* conv_bias, int dtype_w,
                                                   void* conv_tails, int conv_dim, const float* beta0,
                                                   const float* betat, const float* g0, const float* gt, void* out0,
                                                   void* outt, float* states, int B, int L, int Hk, int Hv, int Dk,
                                                   int Dv, int block, int dtype, float scale, int block_begin,
                                                   int block_end, void* stream) {
  const VConv vc = {raw0, rawt, conv_weight, conv_bias, dtype_w, conv_tails, conv_dim};
  return state_fork(qk0, qkt, stride_b, stride_t, beta0, betat, g0, gt, out0, outt, states, B, L, Hk, Hv, Dk, Dv,
                    block, dtype, scale, block_begin, block_end, stream, &vc);
}

extern "C" int dllm_set_fork_split(int mode) {
  if (mode < 0 || mode > 2) return fail(DLLM_EINVAL, "fork split mode %d (0 auto, 1 never, 2 always)", mode);
  return g_fork_split.exchange(mode);
}

extern "C" int dllm_set_spin_limit(int limit) {
  if (limit < 0) return fail(DLLM_EINVAL, "spin limit %d < 0", limit);
  return g_spin_limit.exchange(limit);
}

extern "C" int dllm_status(int reset) {
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "dllm_status: %s", hipGetErrorString(e));
  unsigned v = 0;
  e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(dllm_status_word), sizeof(v), 0, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "dllm_status: %s", hipGetErrorString(e));
  if (reset) {
    const unsigned z = 0;
    e = hipMemcpyToSymbol(HIP_SYMBOL(dllm_status_word), &z, sizeof(z), 0, hipMemcpyHostToDevice);
    if (e != hipSuccess) return fail(DLLM_ELAUNCH, "dllm_status: %s", hipGetErrorString(e));
  }
  return (int)(v & 0x7fffffffu);
}

extern "C" int dllm_set_wait_test_mode(int on) {
  return g_wait_bias.exchange(on ? (1 << 30) : 0) != 0;
}
