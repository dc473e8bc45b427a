// Chunked gated delta rule with per-chunk states and the fused state fork (gfx950 / CDNA4).
//
// One workgroup (4 wavefronts) owns one (sequence b, value head hv, 64-column Dv window) and walks
// the sequence in 32-row tiles. A tile holds `sub` real tokens (sub = gcd(chunk, 32)); the rest
// are zero rows, which are exact no-ops of the recurrence (k = q = v = 0, beta = 0, g = 0).
//
// Per tile, for each stream (clean; plus noised in fork mode):
//   load    q, k (key head hv / (Hv/Hk): GQA by indexing, no expansion), v, beta, g;
//           l2norm + Dk^-1/2 in fp32; gamma = sequential cumsum of g; operands into LDS.
//   G       K^K^T and Q^K^T on MFMA; decay/beta masks -> A (fp32), P.
//   T       T = (I + A)^-1 in fp32 by a blocked inverse (8x8 diagonal blocks by forward
//           substitution, then 8x8 and 16x16 off-diagonal blocks by products), entirely inside the
//           wavefront that produced A; T1 = T diag(beta e^gamma), T2 = T diag(beta).
//   W       W = T1 K^ (= (I+A)^-1 (beta K^ e^gamma)) on MFMA, written over K^.
//   state   clean wave: U = T2 V, V' = U - W S, O = e^gamma (Q^ S) + P V',
//           S <- e^gamma_last S + K^T (e^(gamma_last - gamma) V'), snapshot S every chunk;
//           noised wave (fork): the same O with the noised tile's operands and the clean state
//           before the tile, which the clean wave publishes through LDS.
// The recurrent state S (Dk x 32 columns per wave) lives in fp32 MFMA accumulators for the whole
// sequence and is fed back as the B operand directly from the accumulator layout (rho order).
#include <type_traits>

#include "common.h"

namespace dllm {

struct GdnStream {
  const void* q;
  const void* k;
  const void* v;
  const float* beta;
  const float* g;
  void* out;
  long long q_sb, q_st, q_sh;
  long long k_sb, k_st, k_sh;
  long long v_sb, v_st, v_sh;
  long long b_sb, b_st, b_sh;
  long long g_sb, g_st, g_sh;
};

struct GdnArgs {
  GdnStream s[2];
  const float* init;  // [B, Hv, Dk, Dv] fp32 or null
  float* states;      // [B, T/chunk, Hv, Dk, Dv] fp32 or null
  int B, T, Hk, Hv, Dk, Dv;
  int sub;         // real rows per 32-row tile
  int snap_every;  // tiles per chunk
  float scale;     // applied to q after l2norm
  int l2norm;
  int vec_qk;      // q/k rows: 16-byte vector loads (aligned, Dk equal to the kernel width)
  int vec_v;       // v rows: 16-byte vector loads (aligned, Dv a multiple of 64)
};

// Linear workgroup id such that consecutive ids run on the same XCD (dispatch is round-robin over
// the 8 XCDs): workgroups sharing a key head then share that XCD's L2.
__device__ __forceinline__ int xcd_linear_id(int bid, int n) {
  const int q = n >> 3, r = n & 7, x = bid & 7, i = bid >> 3;
  return (x < r) ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
}

template <int DK, bool BF16, bool FORK>
struct GdnSmem {
  using OpT = typename std::conditional<BF16, bf16, float>::type;
  static constexpr int NS = FORK ? 2 : 1;
  static constexpr int KT = DK / 32;
  static constexpr int QROW = DK + (BF16 ? 8 : 4);  // [32][DK] row stride (elements)
  static constexpr int TROW = 32 + (BF16 ? 8 : 4);  // [.][32] row stride (elements)
  // per-stream byte offsets
  static constexpr int O_QH = 0;
  static constexpr int O_KH = O_QH + 32 * QROW * (int)sizeof(OpT);
  static constexpr int O_KT = O_KH + 32 * QROW * (int)sizeof(OpT);
  static constexpr int O_VT = O_KT + DK * TROW * (int)sizeof(OpT);
  static constexpr int O_P = O_VT + 64 * TROW * (int)sizeof(OpT);
  static constexpr int O_T1 = O_P + 32 * TROW * (int)sizeof(OpT);
  static constexpr int O_T2 = O_T1 + 32 * TROW * (int)sizeof(OpT);
  static constexpr int O_AF = O_T2 + 32 * TROW * (int)sizeof(OpT);
  static constexpr int O_TF = O_AF + 32 * 33 * 4;
  static constexpr int O_YF = O_TF + 32 * 33 * 4;
  static constexpr int O_VEC = O_YF + 16 * 17 * 4;  // gam, bet, eg, egl (32 floats each)
  static constexpr int STREAM_BYTES = ((O_VEC + 4 * 32 * 4) + 15) & ~15;
  static constexpr int FRAG_BYTES = 16 * (int)sizeof(OpT);
  // state operand fragments published by the clean waves: [buffers][2 slices][KT][64 lanes]
  // (double-buffered in fork mode, where the noised waves read them one tile later)
  static constexpr int O_SB = NS * STREAM_BYTES;
  static constexpr int SB_BYTES = (FORK ? 2 : 1) * 2 * KT * 64 * FRAG_BYTES;
  static constexpr int TOTAL = O_SB + SB_BYTES;
};

// N contiguous elements of a row into 16-byte vector registers (raw input dtype). `valid` of them are
// in range, the rest are zero. Vector loads only when the whole run is in range and aligned.
template <typename V, typename OpT, int N>
__device__ __forceinline__ void load_raw(V* dst, const OpT* src, bool vec, int valid) {
  constexpr int EPV = 16 / (int)sizeof(OpT);
  if (vec) {  // uniform: every lane's run is in range (callers clamp rows), no divergence
#pragma unroll
    for (int i = 0; i < N / EPV; ++i) dst[i] = *(const V*)(src + i * EPV);
  } else {
#pragma unroll
    for (int i = 0; i < N / EPV; ++i)
#pragma unroll
      for (int e = 0; e < EPV; ++e) dst[i][e] = (i * EPV + e < valid) ? src[i * EPV + e] : from_f32<OpT>(0.f);
  }
}

template <int DK, bool BF16, bool FORK>
__global__ __launch_bounds__(256) void gdn_chunk_kernel(GdnArgs a) {
  using SM = GdnSmem<DK, BF16, FORK>;
  using OpT = typename SM::OpT;
  using F = Frag<BF16>;
  constexpr int NS = SM::NS;
  constexpr int KT = SM::KT;
  constexpr int QROW = SM::QROW;
  constexpr int TROW = SM::TROW;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SM::TOTAL];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform values live in SGPRs
  const int lane = tid & 63, h = lane >> 5, l32 = lane & 31;

  const int nsl = (a.Dv + 63) >> 6;
  const int lin = xcd_linear_id(blockIdx.x, gridDim.x);
  const int slice = lin % nsl;
  const int hv = (lin / nsl) % a.Hv;
  const int b = lin / (nsl * a.Hv);
  const int hk = hv / (a.Hv / a.Hk);
  const int col0 = slice * 64;
  const int ntiles = a.T / a.sub;
  const int nsnap = a.T / (a.sub * a.snap_every);

  auto QH = [&](int s) { return (OpT*)(smem + s * SM::STREAM_BYTES + SM::O_QH); };
  auto KH = [&](int s) { return (OpT*)(smem + s * SM::STREAM_BYTES + SM::O_KH); };
  auto KTr = [&](int s) { return (OpT*)(smem + s * SM::STREAM_BYTES + SM::O_KT); };
  auto VT = [&](int s) { return (OpT*)(smem + s * SM::STREAM_BYTES + SM::O_VT); };
  auto PP = [&](int s) { return (OpT*)(smem + s * SM::STREAM_BYTES + SM::O_P); };
  auto T1 = [&](int s) { return (OpT*)(smem + s * SM::STREAM_BYTES + SM::O_T1); };
  auto T2 = [&](int s) { return (OpT*)(smem + s * SM::STREAM_BYTES + SM::O_T2); };
  auto AF = [&](int s) { return (float*)(smem + s * SM::STREAM_BYTES + SM::O_AF); };
  auto TF = [&](int s) { return (float*)(smem + s * SM::STREAM_BYTES + SM::O_TF); };
  auto YF = [&](int s) { return (float*)(smem + s * SM::STREAM_BYTES + SM::O_YF); };
  auto GAM = [&](int s) { return (float*)(smem + s * SM::STREAM_BYTES + SM::O_VEC); };
  auto BET = [&](int s) { return GAM(s) + 32; };
  auto EG = [&](int s) { return GAM(s) + 64; };
  auto EGL = [&](int s) { return GAM(s) + 96; };
  auto SBUF = [&](int buf, int sl, int kt) {
    return (F*)(smem + SM::O_SB) + (((buf * 2 + sl) * KT + kt) * 64 + lane);
  };

  // state-phase roles: wave -> (32-column slice, stream)
  const int my_sl = wave & 1;
  const int role = wave >> 1;  // 0 clean (owns S); 1 noised (fork) or idle
  const int mycol = col0 + my_sl * 32 + l32;
  const bool col_ok = mycol < a.Dv;

  f32x16 S[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) S[t] = zero16();
  if (role == 0) {
    if (a.init && col_ok) {
      const float* src = a.init + ((long long)(b * a.Hv + hv) * a.Dk) * a.Dv + mycol;
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int dk = 32 * t + rho(v, h);
          if (dk < a.Dk) S[t][v] = src[(long long)dk * a.Dv];
        }
    }
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      F f;
      acc_to_frag(S[t], f);
      *SBUF(0, my_sl, t) = f;
    }
  }

  // Raw inputs of one tile, held in registers so that the next tile's global loads are in flight
  // while the current tile computes: thread -> (row lr, 1/8 of the q/k row, 8 v columns).
  constexpr int NE = DK / 8;
  constexpr int EPV = 16 / (int)sizeof(OpT);
  using V16 = typename std::conditional<BF16, bf16x8, f32x4>::type;
  V16 rq[NS][NE / EPV], rk[NS][NE / EPV], rv[NS][8 / EPV];
  float rg[NS], rb[NS];
  const int lr = tid >> 3, lseg = tid & 7;
  const bool lreal = lr < a.sub;  // rows >= sub are zero padding (loaded from row 0, zeroed on use)
  auto issue_loads = [&](int t0) {
    const bool real = lreal;
    const long long tok = t0 + (real ? lr : 0);
    const int e0 = lseg * NE;
    const int valid_qk = real ? max(0, min(NE, a.Dk - e0)) : 0;
    const int c8 = col0 + lseg * 8;
    const int valid_v = real ? max(0, min(8, a.Dv - c8)) : 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const GdnStream& st = a.s[s];
      load_raw<V16, OpT, NE>(rq[s], (const OpT*)st.q + b * st.q_sb + tok * st.q_st + hk * st.q_sh + e0, a.vec_qk,
                             valid_qk);
      load_raw<V16, OpT, NE>(rk[s], (const OpT*)st.k + b * st.k_sb + tok * st.k_st + hk * st.k_sh + e0, a.vec_qk,
                             valid_qk);
      load_raw<V16, OpT, 8>(rv[s], (const OpT*)st.v + b * st.v_sb + tok * st.v_st + hv * st.v_sh + c8, a.vec_v,
                            valid_v);
      rg[s] = 0.f;
      rb[s] = 0.f;
      if (wave == 0 && h == 0 && l32 < a.sub) {
        const long long tk = t0 + l32;
        rg[s] = st.g[b * st.g_sb + tk * st.g_st + hv * st.g_sh];
        rb[s] = st.beta[b * st.b_sb + tk * st.b_st + hv * st.b_sh];
      }
    }
  };
  issue_loads(0);

  for (int c = 0; c < ntiles; ++c) {
    const int t0 = c * a.sub;
    __syncthreads();  // previous tile's state phase is done with every LDS operand

    // ------------------------------------------------------------------ load phase (registers -> LDS)
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      {
        const int e0 = lseg * NE;
        float x[NE];
#pragma unroll
        for (int i = 0; i < NE; ++i) x[i] = lreal ? to_f32(rq[s][i / EPV][i % EPV]) : 0.f;
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NE; ++i) ss = __builtin_fmaf(x[i], x[i], ss);
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        ss += __shfl_xor(ss, 4);
        float rn = a.l2norm ? rsqrtf(ss + 1e-6f) : 1.f;
        OpT* qh = QH(s) + lr * QROW + e0;
#pragma unroll
        for (int i = 0; i < NE; ++i) qh[i] = from_f32<OpT>((x[i] * rn) * a.scale);
#pragma unroll
        for (int i = 0; i < NE; ++i) x[i] = lreal ? to_f32(rk[s][i / EPV][i % EPV]) : 0.f;
        ss = 0.f;
#pragma unroll
        for (int i = 0; i < NE; ++i) ss = __builtin_fmaf(x[i], x[i], ss);
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        ss += __shfl_xor(ss, 4);
        rn = a.l2norm ? rsqrtf(ss + 1e-6f) : 1.f;
        OpT* kh = KH(s) + lr * QROW + e0;
        OpT* kt = KTr(s) + e0 * TROW + lr;
#pragma unroll
        for (int i = 0; i < NE; ++i) {
          const OpT y = from_f32<OpT>(x[i] * rn);
          kh[i] = y;
          kt[i * TROW] = y;
        }
        OpT* vt = VT(s) + (lseg * 8) * TROW + lr;
#pragma unroll
        for (int i = 0; i < 8; ++i) vt[i * TROW] = lreal ? rv[s][i / EPV][i % EPV] : from_f32<OpT>(0.f);
      }
      // beta, g and the cumulative decay (sequential order, as a cumsum)
      if (wave == 0) {
        const int r = l32;
        float gam = 0.f;
        for (int q = 0; q < 32; ++q) {
          const float gq = __shfl(rg[s], q, 64);
          if (q <= r) gam += gq;
        }
        const float glast = __shfl(gam, 31, 64);
        if (h == 0) {
          GAM(s)[r] = gam;
          BET(s)[r] = rb[s];
          EG(s)[r] = expf(gam);
          EGL(s)[r] = expf(glast - gam);
        }
      }
    }
    __syncthreads();
    if (c + 1 < ntiles) issue_loads(t0 + a.sub);  // next tile's inputs travel during this tile

    // ------------------------------------------------------------------ G (+ T) phase
    {
      const int gs = FORK ? (wave & 1) : 0;
      const bool isG = FORK ? (wave < 2) : (wave == 0);
      const bool isQK = FORK ? (wave >= 2) : (wave == 1);
      if (isG || isQK) {
        const OpT* X = isG ? KH(gs) : QH(gs);
        const OpT* Kr = KH(gs);
        f32x16 acc = zero16();
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          F fa, fb;
          lds_frag(X + l32 * QROW + kt * 32, h, fa);
          lds_frag(Kr + l32 * QROW + kt * 32, h, fb);
          mma32(acc, fa, fb);
        }
        const float* gam = GAM(gs);
        const float gj = gam[l32];
        if (isG) {
          const float* bet = BET(gs);
          float* Af = AF(gs);
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int i = rho(v, h);
            Af[i * 33 + l32] = (l32 < i) ? bet[i] * acc[v] * expf(gam[i] - gj) : 0.f;
          }
        } else {
          OpT* P = PP(gs);
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int i = rho(v, h);
            P[i * TROW + l32] = from_f32<OpT>((l32 <= i) ? acc[v] * expf(gam[i] - gj) : 0.f);
          }
        }
      }
      if (isG) {
        // T = (I + A)^-1, fp32, inside this wavefront
        const float* Af = AF(gs);
        float* Tf = TF(gs);
        float* Yf = YF(gs);
#pragma unroll
        for (int m = 0; m < 16; ++m) Tf[(m * 2 + h) * 33 + l32] = 0.f;
        wave_lds_sync();
        // level 0: four 8x8 diagonal blocks, one column per lane (lanes 0..31)
        if (h == 0) {
          const int bb = l32 >> 3, cc = l32 & 7, o = 8 * bb;
          float x[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = (i == cc) ? 1.f : 0.f;
#pragma unroll
          for (int i = 1; i < 8; ++i) {
            float sacc = 0.f;
#pragma unroll
            for (int j = 0; j < i; ++j) sacc = __builtin_fmaf(Af[(o + i) * 33 + o + j], x[j], sacc);
            if (i > cc) x[i] = -sacc;
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) Tf[(o + i) * 33 + o + cc] = x[i];
        }
        wave_lds_sync();
        // level 1: T[m+1][m] = -D[m+1] A[m+1][m] D[m] for the three sub-diagonal 8x8 blocks
        {
          const int ii = lane >> 3, jj = lane & 7;
          float y[3];
#pragma unroll
          for (int m = 0; m < 3; ++m) {
            float sacc = 0.f;
#pragma unroll
            for (int kk = 0; kk < 8; ++kk)
              sacc = __builtin_fmaf(Af[(8 * (m + 1) + ii) * 33 + 8 * m + kk], Tf[(8 * m + kk) * 33 + 8 * m + jj], sacc);
            y[m] = sacc;
          }
#pragma unroll
          for (int m = 0; m < 3; ++m) Yf[m * 64 + ii * 8 + jj] = y[m];
          wave_lds_sync();
#pragma unroll
          for (int m = 0; m < 3; ++m) {
            float sacc = 0.f;
#pragma unroll
            for (int kk = 0; kk < 8; ++kk)
              sacc = __builtin_fmaf(Tf[(8 * (m + 1) + ii) * 33 + 8 * (m + 1) + kk], Yf[m * 64 + kk * 8 + jj], sacc);
            y[m] = -sacc;
          }
          wave_lds_sync();  // every lane has read Yf and the diagonal blocks
#pragma unroll
          for (int m = 0; m < 3; ++m) Tf[(8 * (m + 1) + ii) * 33 + 8 * m + jj] = y[m];
        }
        wave_lds_sync();
        // level 2: T[16:32][0:16] = -T16_1 A[16:32][0:16] T16_0
        {
          const int ii = lane >> 2, j4 = (lane & 3) * 4;
          float y[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < 16; ++kk) {
            const float av = Af[(16 + ii) * 33 + kk];
#pragma unroll
            for (int q = 0; q < 4; ++q) y[q] = __builtin_fmaf(av, Tf[kk * 33 + j4 + q], y[q]);
          }
#pragma unroll
          for (int q = 0; q < 4; ++q) Yf[ii * 17 + j4 + q] = y[q];
          wave_lds_sync();
          float z[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < 16; ++kk) {
            const float tv = Tf[(16 + ii) * 33 + 16 + kk];
#pragma unroll
            for (int q = 0; q < 4; ++q) z[q] = __builtin_fmaf(tv, Yf[kk * 17 + j4 + q], z[q]);
          }
          wave_lds_sync();
#pragma unroll
          for (int q = 0; q < 4; ++q) Tf[(16 + ii) * 33 + j4 + q] = -z[q];
        }
        wave_lds_sync();
        // scaled operand copies: T1 = T diag(beta e^gamma), T2 = T diag(beta)
        {
          const float* bet = BET(gs);
          const float* eg = EG(gs);
          OpT* t1 = T1(gs);
          OpT* t2 = T2(gs);
          const float bj = bet[l32], bej = bet[l32] * eg[l32];
#pragma unroll
          for (int m = 0; m < 16; ++m) {
            const int i = 2 * m + h;
            const float tv = (l32 <= i) ? Tf[i * 33 + l32] : 0.f;
            t1[i * TROW + l32] = from_f32<OpT>(tv * bej);
            t2[i * TROW + l32] = from_f32<OpT>(tv * bj);
          }
        }
      }
    }
    __syncthreads();

    // ------------------------------------------------------------------ W phase: W = T1 K^
    {
      constexpr int NT = NS * KT;
#pragma unroll
      for (int id0 = 0; id0 < NT; id0 += 4) {
        const int id = id0 + wave;
        if (id < NT) {
          const int s = id / KT, kt = id % KT;
          F fa, fb;
          lds_frag(T1(s) + l32 * TROW, h, fa);
          lds_frag(KTr(s) + (kt * 32 + l32) * TROW, h, fb);
          f32x16 acc = zero16();
          mma32(acc, fa, fb);
          OpT* W = KH(s);  // K^ row-major is dead after the G phase
#pragma unroll
          for (int v = 0; v < 16; ++v) W[rho(v, h) * QROW + kt * 32 + l32] = from_f32<OpT>(acc[v]);
        }
      }
    }
    __syncthreads();

    // ------------------------------------------------------------------ state phase
    if (role == 0 || FORK) {
      const int s = role;  // stream
      const int sbuf = FORK ? (c & 1) : 0;
      f32x16 accU = zero16(), accWS = zero16(), accQS = zero16();
      {
        F fa, fb;
        lds_frag(T2(s) + l32 * TROW, h, fa);
        lds_frag(VT(s) + (my_sl * 32 + l32) * TROW, h, fb);
        mma32(accU, fa, fb);
      }
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        F fw, fq;
        lds_frag(KH(s) + l32 * QROW + kt * 32, h, fw);
        lds_frag(QH(s) + l32 * QROW + kt * 32, h, fq);
        const F sx = *SBUF(sbuf, my_sl, kt);
        mma32(accWS, fw, sx);
        mma32(accQS, fq, sx);
      }
      const float* eg = EG(s);
      f32x16 vn;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        vn[v] = accU[v] - accWS[v];
        accQS[v] *= eg[rho(v, h)];
      }
      F fv;
      acc_to_frag(vn, fv);
      {
        F fp;
        lds_frag(PP(s) + l32 * TROW, h, fp);
        mma32(accQS, fp, fv);
      }
      // output rows of the real tokens
      if (col_ok) {
        const long long rs = (long long)a.Hv * a.Dv;  // token stride of out
        OpT* ob = (OpT*)a.s[s].out + ((long long)b * a.T + t0) * rs + (long long)hv * a.Dv + col0 + my_sl * 32;
        const unsigned lo = (unsigned)(4 * h) * (unsigned)rs + (unsigned)l32;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int ru = ((v >> 2) << 3) + (v & 3);  // row = ru + 4h
          if (ru + 4 * h < a.sub) (ob + ru * rs)[lo] = from_f32<OpT>(accQS[v]);
        }
      }
      if (role == 0) {
        const float* egl = EGL(s);
        const float lam = eg[31];
        f32x16 vd;
#pragma unroll
        for (int v = 0; v < 16; ++v) vd[v] = vn[v] * egl[rho(v, h)];
        F fd;
        acc_to_frag(vd, fd);
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
          for (int v = 0; v < 16; ++v) S[kt][v] *= lam;
          F fk;
          lds_frag(KTr(s) + (kt * 32 + l32) * TROW, h, fk);
          mma32(S[kt], fk, fd);
        }
        if (a.states && ((c + 1) % a.snap_every) == 0 && col_ok) {
          const int sn = (c + 1) / a.snap_every - 1;
          float* sb = a.states + (((long long)b * nsnap + sn) * a.Hv + hv) * (long long)a.Dk * a.Dv + col0 + my_sl * 32;
          const unsigned lo = (unsigned)(4 * h * a.Dv + l32);
#pragma unroll
          for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int du = 32 * kt + ((v >> 2) << 3) + (v & 3);  // dk = du + 4h
              if (du + 4 * h < a.Dk) __builtin_nontemporal_store(S[kt][v], (sb + (long long)du * a.Dv) + lo);
            }
        }
#pragma unroll
        for (int t = 0; t < KT; ++t) {
          F f;
          acc_to_frag(S[t], f);
          *SBUF(FORK ? ((c + 1) & 1) : 0, my_sl, t) = f;
        }
      }
    }
  }
}

template <int DK, bool BF16, bool FORK>
static int launch_gdn(const GdnArgs& a, hipStream_t st) {
  const int nsl = (a.Dv + 63) / 64;
  const long long nblk = (long long)a.B * a.Hv * nsl;
  if (nblk > 0x7fffffff) return fail(DLLM_EUNSUPPORTED, "gdn: grid too large");
  gdn_chunk_kernel<DK, BF16, FORK><<<dim3((unsigned)nblk), dim3(256), 0, st>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "gdn launch: %s", hipGetErrorString(e));
  return DLLM_OK;
}

static int gcd_int(int x, int y) {
  while (y) { int t = x % y; x = y; y = t; }
  return x;
}

static int dispatch_gdn(GdnArgs& a, int dtype, bool fork, hipStream_t st) {
  const int dk = a.Dk <= 64 ? 64 : 128;
  if (a.Dk > 128) return fail(DLLM_EUNSUPPORTED, "gdn: Dk=%d > 128 not supported", a.Dk);
  if (dtype == DT_BF16) {
    if (dk == 64) return fork ? launch_gdn<64, true, true>(a, st) : launch_gdn<64, true, false>(a, st);
    return fork ? launch_gdn<128, true, true>(a, st) : launch_gdn<128, true, false>(a, st);
  }
  if (dtype == DT_F32) {
    if (dk == 64) return fork ? launch_gdn<64, false, true>(a, st) : launch_gdn<64, false, false>(a, st);
    if (fork) return fail(DLLM_EUNSUPPORTED, "gdn: fused fork needs Dk<=64 in fp32 (use the two-pass fork)");
    return launch_gdn<128, false, false>(a, st);
  }
  return fail(DLLM_EUNSUPPORTED, "gdn: dtype %d not supported", dtype);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace dllm

using namespace dllm;

extern "C" int dllm_gdn_fused_fork_supported(int Dk, int block, int dtype) {
  if (block <= 0 || 32 % block != 0) return 0;
  if (Dk <= 0 || Dk > 128) return 0;
  if (dtype == DT_F32 && Dk > 64) return 0;
  return dtype == DT_F32 || dtype == DT_BF16;
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
  GdnArgs a = {};
  GdnStream& s = a.s[0];
  s.q = q; s.k = k; s.v = v; s.g = g; s.beta = beta; s.out = out;
  s.q_sb = q_strides[0]; s.q_st = q_strides[1]; s.q_sh = q_strides[2];
  s.k_sb = k_strides[0]; s.k_st = k_strides[1]; s.k_sh = k_strides[2];
  s.v_sb = v_strides[0]; s.v_st = v_strides[1]; s.v_sh = v_strides[2];
  s.g_sb = g_strides[0]; s.g_st = g_strides[1]; s.g_sh = g_strides[2];
  s.b_sb = beta_strides[0]; s.b_st = beta_strides[1]; s.b_sh = beta_strides[2];
  a.init = initial_state;
  a.states = states;
  a.B = B; a.T = T; a.Hk = Hk; a.Hv = Hv; a.Dk = Dk; a.Dv = Dv;
  a.sub = gcd_int(chunk, 32);
  a.snap_every = chunk / a.sub;
  a.scale = scale;
  a.l2norm = use_qk_l2norm;
  const int esz = dtype == DT_BF16 ? 2 : 4;
  const int vel = 16 / esz;
  auto st_ok = [&](const int64_t* st3) { return (st3[0] % vel == 0) && (st3[1] % vel == 0) && (st3[2] % vel == 0); };
  const int dkw = Dk <= 64 ? 64 : 128;
  a.vec_qk = aligned16(q) && aligned16(k) && st_ok(q_strides) && st_ok(k_strides) && Dk == dkw;
  a.vec_v = aligned16(v) && st_ok(v_strides) && (Dv % 64 == 0);
  return dispatch_gdn(a, dtype, false, (hipStream_t)stream);
}

extern "C" int dllm_gdn_state_fork_fwd(const void* qkv0, const void* qkvt, int64_t qkv_stride_b, int64_t qkv_stride_t,
                                       const float* beta0, const float* betat, const float* g0, const float* gt,
                                       void* out0, void* outt, float* states, int B, int L, int Hk, int Hv, int Dk,
                                       int Dv, int block, int dtype, float scale, void* stream) {
  if (!qkv0 || !qkvt || !beta0 || !betat || !g0 || !gt || !out0 || !outt) return fail(DLLM_EINVAL, "gdn fork: null pointer");
  if (B <= 0 || L <= 0 || Hk <= 0 || Hv <= 0 || Dk <= 0 || Dv <= 0 || block <= 0)
    return fail(DLLM_EINVAL, "gdn fork: bad sizes");
  if (L % block) return fail(DLLM_EINVAL, "L=%d is not a multiple of block=%d", L, block);
  if (Hv % Hk) return fail(DLLM_EINVAL, "gdn fork: Hv=%d is not a multiple of Hk=%d", Hv, Hk);
  if (!dllm_gdn_fused_fork_supported(Dk, block, dtype))
    return fail(DLLM_EUNSUPPORTED, "gdn fork: fused fork unsupported for Dk=%d block=%d dtype=%d", Dk, block, dtype);
  GdnArgs a = {};
  const int esz = dtype == DT_BF16 ? 2 : 4;
  const char* base[2] = {(const char*)qkv0, (const char*)qkvt};
  const float* bet[2] = {beta0, betat};
  const float* gg[2] = {g0, gt};
  void* outs[2] = {out0, outt};
  for (int i = 0; i < 2; ++i) {
    GdnStream& s = a.s[i];
    s.q = base[i];
    s.k = base[i] + (long long)Hk * Dk * esz;
    s.v = base[i] + 2LL * Hk * Dk * esz;
    s.q_sb = s.k_sb = s.v_sb = qkv_stride_b;
    s.q_st = s.k_st = s.v_st = qkv_stride_t;
    s.q_sh = s.k_sh = Dk;
    s.v_sh = Dv;
    s.beta = bet[i]; s.b_sb = (long long)L * Hv; s.b_st = Hv; s.b_sh = 1;
    s.g = gg[i]; s.g_sb = (long long)L * Hv; s.g_st = Hv; s.g_sh = 1;
    s.out = outs[i];
  }
  a.init = nullptr;
  a.states = states;
  a.B = B; a.T = L; a.Hk = Hk; a.Hv = Hv; a.Dk = Dk; a.Dv = Dv;
  a.sub = block;
  a.snap_every = 1;
  a.scale = scale;
  a.l2norm = 1;
  const int vel = 16 / esz;
  const bool st_ok = (qkv_stride_b % vel == 0) && (qkv_stride_t % vel == 0) && (Dk % vel == 0) && (Dv % vel == 0) &&
                     ((long long)Hk * Dk % vel == 0);
  const int dkw = Dk <= 64 ? 64 : 128;
  a.vec_qk = aligned16(qkv0) && aligned16(qkvt) && st_ok && Dk == dkw;
  a.vec_v = aligned16(qkv0) && aligned16(qkvt) && st_ok && (Dv % 64 == 0);
  return dispatch_gdn(a, dtype, true, (hipStream_t)stream);
}
