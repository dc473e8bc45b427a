// Projections of a decoding step: y[M, N] = x[M, K] W[N, K]^T with few token rows (M <= 64), bf16
// in and out, fp32 accumulation (gfx950).
//
// A cached denoising step runs every projection of the stack on one block of tokens (32 rows), so
// each weight is read once for 32 rows and the step is bound by streaming the weights from HBM.
//   * Work units. An output tile is 128 features x 32 token rows; a unit is one step of 64 k of one
//     tile (16 KB of weights). The launch has G workgroups, and workgroup w takes the contiguous
//     unit range [w U / G, (w + 1) U / G) of the U units, in tile order. With fewer than two tiles
//     per CU, G is one per CU: every CU streams the same number of bytes whatever the projection's
//     shape (a grid of whole tiles or of K splits leaves CUs idle, or with twice the work of
//     others, at N = 5120). With more tiles (lm_head), G is the tile count: nothing is split.
//   * Per unit the workgroup stages the weight tile [128 features x 64 k] and the token tile
//     [32 rows x 64 k] with direct global -> LDS loads (each wave instruction moves 1 KB: eight
//     whole 128-byte row segments, no registers), in a ring of LIN_NST stages that keeps
//     LIN_NST - 1 units in flight, across tile boundaries. The weights are read non-temporally at
//     device scope (each is read once per step; measured 3.51-3.53 vs 3.67-3.87 ms for a cached
//     denoising step of the 16-layer 27B-class stack, lm_head 254 vs 277 us), the token tile,
//     re-read for every feature tile, with the default policy;
//   * rows are 128 bytes with their 16-byte chunks XOR-swizzled by (row >> 1), so the operand reads
//     (16 rows of one chunk per pass) touch every bank once;
//   * wave w reads the B operand (lane = feature) of its 32 features and the A operand (lane =
//     token) from LDS, 16 bytes each, and issues four v_mfma_f32_32x32x16_bf16 per unit (lane
//     (row, h) carries k = 16u + 8h + 0..7 in MFMA u for both operands);
//   * a tile whose units all belong to one workgroup is rounded to bf16 and stored. A tile split
//     between workgroups leaves an fp32 partial per piece (at most two per workgroup: its first
//     and its last piece); a second kernel sums the pieces in workgroup order (deterministic) for
//     the split tiles only;
//   * more than 32 token rows: the next 32 rows are further tiles (the weights are streamed again);
//   * up to four projections of the same x (q | k | v, the four mixer inputs, gate | up) share one
//     launch: the feature tiles run through the weights in turn. With the SwiGLU epilogue
//     (gate | up) the second kernel writes round(round(silu(gate)) * up), the MLP's activation,
//     over the whole gate projection (whole tiles were stored rounded, the up tiles in the
//     workspace);
//   * the second kernel can also finish what reads the projection next, from the same sums: the
//     residual add and RMSNorm after out_proj / o_proj / down_proj (one workgroup per token row)
//     or, after a Gated DeltaNet layer's four input projections, the short conv and the gates (one
//     block per tile). Either equals the separate launches bit for bit.
#include <algorithm>
#include <mutex>

#include "common.h"

namespace dllm {

constexpr int LIN_NST = 4;                 // ring stages (4 x 20 KB: two workgroups fit a CU)
constexpr int LIN_W_BYTES = 128 * 64 * 2;  // weight tile of one unit
constexpr int LIN_X_BYTES = 32 * 64 * 2;   // token tile of one unit
constexpr int LIN_STAGE = LIN_W_BYTES + LIN_X_BYTES;
constexpr int LIN_TILE = 32 * 128;         // floats of one partial tile
constexpr int LIN_CUS = 256;               // compute units of the chip (MI355X)

__device__ __forceinline__ int lin_off(int row, int chunk) {  // byte offset of a 16-byte chunk of a 128-byte row
  return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4);
}

template <int N>
__device__ __forceinline__ void lin_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// wait until at most `behind` units of PER loads each are in flight (behind <= B)
template <int B, int PER>
__device__ __forceinline__ void lin_wait_behind(int behind) {
  if constexpr (B > 0) {
    if (behind >= B) lin_wait_vmcnt<B * PER>();
    else lin_wait_behind<B - 1, PER>(behind);
  } else {
    lin_wait_vmcnt<0>();
  }
}

constexpr int LIN_MAXSEG = 4;
struct LinSeg {
  const bf16* w;  // [N, K]
  bf16* y;        // [M, N]
  int N;
  int tile0;      // first feature tile of this projection
};
struct LinArgs {
  const bf16* x;
  LinSeg seg[LIN_MAXSEG];
  float* part;    // [G][2][32][128] fp32 partial tiles: a workgroup's first and last piece
  bf16* up;       // swiglu: the up projection's whole tiles [M, N], rounded
  int nseg, M, K;
  int ntn;        // feature tiles over all projections
  int ns;         // units per tile (K / 64)
  int units;      // tiles * ns, tiles = ntn * ceil(M / 32)
  int uq, ur;     // units = uq * G + ur
  int G, swiglu;
};

// First unit of workgroup w, floor(w U / G) = w q + floor(w r / G) with U = q G + r (32-bit: w, r < G
// <= 32768). The workgroup whose range holds unit u: floor(((u + 1) G - 1) / U), the largest w with
// start(w) <= u; the quotient in double is exact here (numerator < 2^46, and a quotient just below
// an integer k <= G is at least 1/U >= 2^-31 below it, far more than a double's spacing near k).
__device__ __forceinline__ int lin_start(const LinArgs& a, int w) { return w * a.uq + (w * a.ur) / a.G; }
__device__ __forceinline__ int lin_owner(const LinArgs& a, int u) {
  return (int)(((double)(u + 1) * a.G - 1.0) / (double)a.units);
}
__device__ __forceinline__ int lin_seg(const LinArgs& a, int nt) {  // projection of feature tile nt
  int si = 0;
#pragma unroll
  for (int i = 1; i < LIN_MAXSEG; ++i)
    if (i < a.nseg && nt >= a.seg[i].tile0) si = i;
  return si;
}

__global__ __launch_bounds__(256) void decode_linear_kernel(LinArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[LIN_NST * LIN_STAGE];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int u0 = lin_start(a, blockIdx.x);
  const int nunits = lin_start(a, blockIdx.x + 1) - u0;
  const bf16* __restrict__ const x = a.x;
  const int M = a.M, K = a.K, ns = a.ns;

  // staging role of this lane: row 8 i + lane / 8 of its rows, logical chunk (lane % 8) ^ key(row)
  const int srow = lane >> 3, schunk = lane & 7;
  int st_tile = u0 / ns, st_step = u0 - st_tile * ns;  // unit the next stage() call loads
  auto stage = [&](int j) {  // unit u0 + j into ring slot j % LIN_NST
    const int mt = st_tile / a.ntn, nt = st_tile - mt * a.ntn;
    const LinSeg& sg = a.seg[lin_seg(a, nt)];
    const int n0 = (nt - sg.tile0) * 128, m0 = mt * 32, k0 = 64 * st_step;
    unsigned char* sb = smem + (j % LIN_NST) * LIN_STAGE;
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // this wave's 4 of the 16 weight instructions: rows 32 wave + 8 i ..
      const int row = 32 * wave + 8 * i + srow;
      const int n = min(n0 + row, sg.N - 1);  // rows past N load a valid row; their outputs are not stored
      const int c = schunk ^ ((row >> 1) & 7);
      dma_load16_stream(sg.w + (long long)n * K + k0 + 8 * c, sb + (32 * wave + 8 * i) * 128);
    }
    {  // token tile: wave w stages rows 8 w .. 8 w + 7
      const int row = 8 * wave + srow;
      const int m = min(m0 + row, M - 1);
      const int c = schunk ^ ((row >> 1) & 7);
      dma_load16(x + (long long)m * K + k0 + 8 * c, sb + LIN_W_BYTES + 8 * wave * 128);
    }
    if (++st_step == ns) st_step = 0, ++st_tile;
  };
  constexpr int PER = 5;  // direct loads per wave per unit
  static_assert(LIN_NST >= 2 && LIN_NST * LIN_STAGE <= 160 * 1024, "ring depth");
  // unit j has landed for this wave; the units issued after it may still travel
  auto wait_unit = [&](int j) { lin_wait_behind<LIN_NST - 2, PER>(min(LIN_NST - 2, nunits - 1 - j)); };

  // acc: lane holds feature column l32 of this wave's 32 features, token rows rho(v, h)
  auto flush = [&](int tile, bool whole, int slot, const f32x16& acc) {
    const int mt = tile / a.ntn, nt = tile - mt * a.ntn;
    const int si = lin_seg(a, nt);
    const LinSeg& sg = a.seg[si];
    if (whole) {
      const int n = (nt - sg.tile0) * 128 + 32 * wave + l32;
      bf16* const y = (a.swiglu && si == 1) ? a.up : sg.y;
      if (n >= sg.N) return;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = mt * 32 + rho(v, h);
        if (m < M) y[(long long)m * sg.N + n] = (bf16)acc[v];
      }
    } else {
      float* const p = a.part + (long long)(2 * blockIdx.x + slot) * LIN_TILE + 32 * wave + l32;
#pragma unroll
      for (int v = 0; v < 16; ++v) p[rho(v, h) * 128] = acc[v];
    }
  };

  f32x16 acc = zero16();
#pragma unroll
  for (int j = 0; j < LIN_NST - 1; ++j)
    if (j < nunits) stage(j);
  if (nunits > 0) wait_unit(0);
  __syncthreads();
  int tile = u0 / ns, step = u0 - tile * ns;
  int pstep0 = step, slot = 0;  // step the current piece began at; partial slot of the piece
  for (int j = 0; j < nunits; ++j) {
    if (j + LIN_NST - 1 < nunits) stage(j + LIN_NST - 1);  // its slot held unit j - 1, done before the barrier
    const unsigned char* sb = smem + (j % LIN_NST) * LIN_STAGE;
    const unsigned char* xs = sb + LIN_W_BYTES;
    bf16x8 av[4], bv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      av[u] = *(const bf16x8*)(xs + lin_off(l32, 2 * u + h));
      bv[u] = *(const bf16x8*)(sb + lin_off(32 * wave + l32, 2 * u + h));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[u], bv[u], acc, 0, 0, 0);
    if (step == ns - 1 || j == nunits - 1) {  // the piece ends: the tile's last unit or the range's
      flush(tile, pstep0 == 0 && step == ns - 1, slot, acc);
      acc = zero16();
      slot = 1;
      pstep0 = 0;
    }
    if (++step == ns) step = 0, ++tile;
    if (j + 1 < nunits) wait_unit(j + 1);
    __syncthreads();  // unit j + 1 staged by every wave; every wave is done with unit j's stage
  }
}

// Sum of a tile's pieces at elements 4 q .. 4 q + 3 (row q / 32, columns 4 (q % 32) ..) in
// workgroup order: the pieces of its owners w0..w1. A piece is its workgroup's first (slot 0) unless
// the workgroup began in an earlier tile, which only the first owner can have (then the piece is
// its last, slot 1). The pieces' 16-byte loads go out eight at a time before their sums.
__device__ __forceinline__ f32x4 lin_sum_pieces(const LinArgs& a, int t0, int w0, int w1, int q) {
  const f32x4* const p = (const f32x4*)a.part + q;
  constexpr int T4 = LIN_TILE / 4;
  f32x4 s = p[(long long)(2 * w0 + (lin_start(a, w0) >= t0 ? 0 : 1)) * T4];
  for (int wb = w0 + 1; wb <= w1; wb += 8) {
    f32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (wb + i <= w1) v[i] = p[(long long)(2 * (wb + i)) * T4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (wb + i <= w1) s += v[i];
  }
  return s;
}

constexpr int LIN_FIXMAX = 512;
struct LinFix {
  int n;                   // split tiles in this launch
  int tile[LIN_FIXMAX];
};
constexpr int LIN_FIX_CHUNKS = LIN_TILE / 4 / 256;  // blocks per tile: one float4 per thread

// Tiles split between workgroups (listed by the host): block (i, c) sums chunk c of tile i's pieces.
__global__ __launch_bounds__(256) void decode_linear_fixup_kernel(LinArgs a, LinFix f) {
  const int tile = f.tile[blockIdx.x];
  const int t0 = tile * a.ns, w0 = lin_owner(a, t0), w1 = lin_owner(a, t0 + a.ns - 1);
  const int mt = tile / a.ntn, nt = tile - mt * a.ntn;
  const LinSeg& sg = a.seg[lin_seg(a, nt)];
  const int q = blockIdx.y * 256 + threadIdx.x;
  const f32x4 s = lin_sum_pieces(a, t0, w0, w1, q);
  const int m = mt * 32 + (q >> 5), n = (nt - sg.tile0) * 128 + 4 * (q & 31);
  if (m >= a.M) return;
  bf16* const y = sg.y + (long long)m * sg.N;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (n + i < sg.N) y[n + i] = (bf16)s[i];
}

// The Gated DeltaNet layer's input projections (in_proj_qkv | in_proj_z | in_proj_b | in_proj_a)
// of a decoding step, finished together with the short conv and the gates that read them.
struct GdnPrologue {
  const bf16* prefix;  // [sequences, C, P]: the conv carry-in (the prefix's last P projections), or null
  const void* conv_w;  // [C, width]
  const void* conv_b;  // [C] or null
  bf16* mixed;         // [M, C]: conv + SiLU of the qkv projection
  const void* a_log;   // [H]
  const void* dt_bias;  // [H]
  float* beta;         // [M, H]
  float* g;            // [M, H]
  int T;               // tokens per sequence (divides 32): row m is token m % T of sequence m / T
  int width, P;        // conv width; carry-in length (0 or width - 1)
};

// One block per output tile (32 rows x 128 features): the tile's rounded values (stored whole by
// the streaming kernel, or its pieces summed in workgroup order and stored, as the fixup does; all
// of a thread's loads go out before their sums) go to LDS, then by projection:
//   qkv: the causal depthwise conv + SiLU (width KW) of every (row, channel) of the tile, as the
//        generic conv kernel computes it: taps in order from the oldest, inputs rounded through the
//        weight type, the sum and the SiLU rounded. A thread walks a run of up to 16 rows of one
//        channel inside one sequence (a tile holds whole sequences) with the last KW - 1 inputs in
//        registers: before the run they are the tile's earlier rows or, at a sequence's start, the
//        carry-in, loaded (with the channel's weights) before the tile's values;
//   z:   nothing more (whole tiles take no block work at all);
//   b:   beta = round(sigmoid(b)), a:   g = -exp(A_log) softplus(a + dt_bias), as the gates kernel,
//        each thread one head column (its A_log and dt_bias loaded before the tile's values).
template <typename TW, typename TP, int KW>
__global__ __launch_bounds__(256) void decode_gdn_prologue_kernel(LinArgs a, GdnPrologue p) {
  static_assert(KW >= 2 && KW <= 8, "conv width");
  __shared__ float vals[32][129];
  const int tile = blockIdx.x;
  const int mt = tile / a.ntn, nt = tile - mt * a.ntn;
  const int si = lin_seg(a, nt);
  const LinSeg& sg = a.seg[si];
  const int n0 = (nt - sg.tile0) * 128;
  const int t0 = tile * a.ns;
  const int w0 = lin_owner(a, t0), w1 = lin_owner(a, t0 + a.ns - 1);
  const bool split = w0 != w1;
  if (si == 1 && !split) return;
  const int cl0 = threadIdx.x & 127;
  // conv runs: item = run * 128 + channel, run j covering tile rows [j rl, (j + 1) rl); this thread
  // takes items tid, tid + 256, ..
  const int rl = p.T < 16 ? p.T : 16;  // rows per run
  const int nitems = 128 * (32 / rl);
  float wv[KW], pre[KW - 1], bv = 0.f;
  auto run_rows = [&](int item, int& row0, int& pos0) {
    row0 = (item >> 7) * rl;
    pos0 = (mt * 32 + row0) % p.T;
  };
  auto load_pre = [&](int item, float* h) {  // carry-in of the run's sequence (its first run only)
    int row0, pos0;
    run_rows(item, row0, pos0);
    const long long seq = (mt * 32 + row0) / p.T;
#pragma unroll
    for (int j = 0; j < KW - 1; ++j) {
      const int u = pos0 - (KW - 1) + j;  // position of tap j before the run's first row
      h[j] = (u < 0 && p.P) ? round_through<TW>((float)p.prefix[(seq * sg.N + n0 + (item & 127)) * p.P + (p.P + u)])
                            : 0.f;
    }
  };
  if (si == 0 && n0 + cl0 < sg.N) {
    const TW* const w = (const TW*)p.conv_w + (long long)(n0 + cl0) * KW;
#pragma unroll
    for (int j = 0; j < KW; ++j) wv[j] = to_f32(w[j]);
    bv = p.conv_b ? to_f32(((const TW*)p.conv_b)[n0 + cl0]) : 0.f;
    if ((int)threadIdx.x < nitems) load_pre(threadIdx.x, pre);
  }
  // gates: the head column n0 + cl0 of this thread
  float dtb = 0.f, nea = 0.f;
  if (si == 3 && n0 + cl0 < sg.N) {
    dtb = to_f32(((const TP*)p.dt_bias)[n0 + cl0]);
    nea = -expf(to_f32(((const TP*)p.a_log)[n0 + cl0]));
  }
  constexpr int KQ = LIN_TILE / 4 / 256;  // float4 slots per thread: q = k 256 + tid, row q / 32, features 4 (q % 32) ..
  if (split) {
    constexpr int T4 = LIN_TILE / 4;
    const f32x4* const pp = (const f32x4*)a.part + threadIdx.x;
    const long long first = (long long)(2 * w0 + (lin_start(a, w0) >= t0 ? 0 : 1)) * T4;
    f32x4 sum[KQ];
#pragma unroll
    for (int k = 0; k < KQ; ++k) sum[k] = pp[first + 256 * k];
    for (int wb = w0 + 1; wb <= w1; wb += 4) {
      f32x4 pc[4][KQ];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (wb + i <= w1)
#pragma unroll
          for (int k = 0; k < KQ; ++k) pc[i][k] = pp[(long long)(2 * (wb + i)) * T4 + 256 * k];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (wb + i <= w1)
#pragma unroll
          for (int k = 0; k < KQ; ++k) sum[k] += pc[i][k];
    }
#pragma unroll
    for (int k = 0; k < KQ; ++k) {
      const int q = k * 256 + threadIdx.x;
      const int r = q >> 5, c = (q & 31) * 4;
      const int m = mt * 32 + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = round_through<bf16>(sum[k][e]);
        vals[r][c + e] = v;
        if (m < a.M && n0 + c + e < sg.N) sg.y[(long long)m * sg.N + n0 + c + e] = (bf16)v;
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < KQ; ++k) {
      const int q = k * 256 + threadIdx.x;
      const int r = q >> 5, c = (q & 31) * 4;
      const int m = mt * 32 + r;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        vals[r][c + e] = (m < a.M && n0 + c + e < sg.N) ? (float)sg.y[(long long)m * sg.N + n0 + c + e] : 0.f;
    }
  }
  if (si == 1) return;
  __syncthreads();
  if (si == 0) {
    for (int item = threadIdx.x; item < nitems; item += 256) {
      const int cl = item & 127;
      const int n = n0 + cl;
      int row0, pos0;
      run_rows(item, row0, pos0);
      if (n >= sg.N || mt * 32 + row0 >= a.M) continue;
      float h[KW - 1];
      if (item != (int)threadIdx.x) load_pre(item, h);
      else
#pragma unroll
        for (int j = 0; j < KW - 1; ++j) h[j] = pre[j];
#pragma unroll
      for (int j = 0; j < KW - 1; ++j) {  // taps inside the sequence before the run: the tile's rows
        const int u = pos0 - (KW - 1) + j;
        if (u >= 0) h[j] = round_through<TW>(vals[row0 - (KW - 1) + j][cl]);
      }
      bf16* const out = p.mixed + (long long)(mt * 32 + row0) * sg.N + n;
      for (int t = 0; t < rl; ++t) {
        if (mt * 32 + row0 + t >= a.M) break;
        const float xv = round_through<TW>(vals[row0 + t][cl]);
        float acc = bv;
#pragma unroll
        for (int j = 0; j < KW - 1; ++j) acc = __builtin_fmaf(wv[j], h[j], acc);
        acc = __builtin_fmaf(wv[KW - 1], xv, acc);
#pragma unroll
        for (int j = 0; j + 1 < KW - 1; ++j) h[j] = h[j + 1];
        h[KW - 2] = xv;
        acc = round_through<TW>(acc);
        out[(long long)t * sg.N] = (bf16)round_through<TW>(silu_f32(acc));
      }
    }
  } else if (n0 + cl0 < sg.N) {
    for (int r = threadIdx.x >> 7; r < 32; r += 2) {
      const int m = mt * 32 + r;
      if (m >= a.M) break;
      const float x = vals[r][cl0];
      if (si == 2) {
        p.beta[(long long)m * sg.N + n0 + cl0] = round_through<bf16>(1.f / (1.f + expf(-x)));
      } else {
        const float av = x + dtb;
        const float sp = av > 20.f ? av : log1pf(expf(av));
        p.g[(long long)m * sg.N + n0 + cl0] = nea * sp;
      }
    }
  }
}

// SwiGLU epilogue over every gate tile, block (tile, c) for chunk c: y0 = round(round(silu(gate)) *
// up), gate and up each the rounded sum of their tile (stored whole by the main kernel, or summed
// here from the pieces).
__global__ __launch_bounds__(256) void decode_linear_swiglu_kernel(LinArgs a) {
  const int ntg = a.seg[1].tile0;  // gate tiles per 32 token rows
  const int mt = blockIdx.x / ntg, ng = blockIdx.x - mt * ntg;
  const int tg = mt * a.ntn + ng, tu = tg + ntg;
  const int N = a.seg[0].N;
  const int g0 = tg * a.ns, gw0 = lin_owner(a, g0), gw1 = lin_owner(a, g0 + a.ns - 1);
  const int u0 = tu * a.ns, uw0 = lin_owner(a, u0), uw1 = lin_owner(a, u0 + a.ns - 1);
  const int q = blockIdx.y * 256 + threadIdx.x;
  const int m = mt * 32 + (q >> 5), n = ng * 128 + 4 * (q & 31);
  if (m >= a.M) return;
  f32x4 gs = {}, us = {};
  if (gw0 != gw1) gs = lin_sum_pieces(a, g0, gw0, gw1, q);
  if (uw0 != uw1) us = lin_sum_pieces(a, u0, uw0, uw1, q);
  bf16* const y = a.seg[0].y + (long long)m * N;
  const bf16* const up = a.up + (long long)m * N;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (n + i >= N) break;
    const float gv = gw0 == gw1 ? (float)y[n + i] : round_through<bf16>(gs[i]);
    const float uv = uw0 == uw1 ? (float)up[n + i] : round_through<bf16>(us[i]);
    y[n + i] = (bf16)(round_through<bf16>(silu_f32(gv)) * uv);
  }
}

// The end of a projection fused with the residual add and RMSNorm that follow it (the decoder's
// out_proj / o_proj and down_proj, then the next norm), in place of the fixup launch and the norm's
// own: one workgroup per token row m.
//   1. Every thread forms the rounded projection values of 4-feature slots q = tid, tid + blockDim,
//      ..: the tile's stored value (seg[0].y) or, for a tile split between workgroups, the sum of
//      its pieces in workgroup order, rounded (the fixup's arithmetic; the pieces' loads go out
//      eight at a time before their sums), into an LDS row of bf16 (exact: the values are rounded).
//   2. The first nw waves run the row RMSNorm kernel's arithmetic on that row: lane vectors of 8
//      features (vector k nw + wave, lane), s = round(y + r) written to sum_out, sums of squares in
//      lane, wave and wave-order, out = round(s rsqrt(mean(s^2) + eps) (1 + w)) (w as is with
//      unit = 0). Their residual and weight loads are issued before step 1.
template <typename TW, int NVW>
__global__ __launch_bounds__(1024) void decode_linear_rmsnorm_kernel(LinArgs a, const bf16* __restrict__ r,
                                                                     bf16* __restrict__ sum_out,
                                                                     const TW* __restrict__ w, bf16* __restrict__ out,
                                                                     float eps, int unit, int nw) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lin_rms_smem[];
  bf16* const yrow = (bf16*)lin_rms_smem;  // [N]
  float* const part = (float*)(lin_rms_smem + (size_t)a.seg[0].N * sizeof(bf16));  // [8]
  typedef __attribute__((ext_vector_type(8))) TW W8;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int m = blockIdx.x, mt = m >> 5, mr = m & 31;
  const int N = a.seg[0].N;
  const long long base = (long long)m * N;
  const bool norm_wave = wv < nw;
  bf16x8 rv[NVW];
  W8 wt[NVW];
  if (norm_wave) {
#pragma unroll
    for (int k = 0; k < NVW; ++k) {
      const int c0 = ((k * nw + wv) * 64 + lane) * 8;
      wt[k] = *(const W8*)(w + c0);
      rv[k] = *(const bf16x8*)(r + base + c0);
    }
  }
  for (int q = threadIdx.x; q < N / 4; q += blockDim.x) {
    const int c = 4 * q;
    const int t0 = (mt * a.ntn + (c >> 7)) * a.ns;
    const int w0 = lin_owner(a, t0), w1 = lin_owner(a, t0 + a.ns - 1);
    bf16x4 yv;
    if (w0 == w1) {
      yv = *(const bf16x4*)(a.seg[0].y + base + c);
    } else {
      const float* const p = a.part + mr * 128 + (c & 127);
      f32x4 sum = *(const f32x4*)(p + (long long)(2 * w0 + (lin_start(a, w0) >= t0 ? 0 : 1)) * LIN_TILE);
      for (int wb = w0 + 1; wb <= w1; wb += 8) {
        f32x4 pc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (wb + i <= w1) pc[i] = *(const f32x4*)(p + (long long)(2 * (wb + i)) * LIN_TILE);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (wb + i <= w1) sum += pc[i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) yv[i] = (bf16)sum[i];
    }
    *(bf16x4*)(yrow + c) = yv;
  }
  __syncthreads();
  float v[NVW][8];
  if (norm_wave) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NVW; ++k) {
      const int c0 = ((k * nw + wv) * 64 + lane) * 8;
      const bf16x8 yv = *(const bf16x8*)(yrow + c0);
      bf16x8 sv;
#pragma unroll
      for (int i = 0; i < 8; ++i) sv[i] = (bf16)((float)yv[i] + (float)rv[k][i]);
      *(bf16x8*)(sum_out + base + c0) = sv;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v[k][i] = (float)sv[i];
        ss = __builtin_fmaf(v[k][i], v[k][i], ss);
      }
    }
    ss = wave_sum(ss);
    if (lane == 0) part[wv] = ss;
  }
  __syncthreads();
  if (!norm_wave) return;
  float tot = part[0];
  for (int i = 1; i < nw; ++i) tot += part[i];
  const float inv = rsqrtf(tot / (float)N + eps);
#pragma unroll
  for (int k = 0; k < NVW; ++k) {
    const int c0 = ((k * nw + wv) * 64 + lane) * 8;
    bf16x8 yv;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float wf = to_f32(wt[k][i]);
      yv[i] = (bf16)(v[k][i] * inv * (unit ? 1.f + wf : wf));
    }
    *(bf16x8*)(out + base + c0) = yv;
  }
}

}  // namespace dllm

using namespace dllm;

static long long lin_units(int M, long long ntn, int K) { return ntn * ((M + 31) / 32) * (K / 64); }

extern "C" int dllm_decode_linear_workgroups(int M, int N, int K) {
  if (M <= 0 || M > 64 || N <= 0 || K <= 0 || K % 64) return 0;
  const long long tiles = (long long)((N + 127) / 128) * ((M + 31) / 32);
  const long long u = tiles * (K / 64);
  if (u > 0x7fffffffLL) return 0;
  // enough whole tiles to fill the chip twice over: one tile per workgroup, nothing split;
  // otherwise one workgroup per CU, each an equal share of the units
  if (tiles >= 2 * LIN_CUS) return (int)(tiles < 32768 ? tiles : 32768);
  return (int)(u < LIN_CUS ? u : LIN_CUS);
}

extern "C" long long dllm_decode_linear_workspace_bytes(int M, int N_gate, int workgroups, int swiglu) {
  if (M <= 0 || workgroups <= 0 || N_gate < 0) return -1;
  long long b = (long long)workgroups * 2 * LIN_TILE * sizeof(float);
  if (swiglu) b += ((long long)M * N_gate * 2 + 255) / 256 * 256;
  return b;
}

// Checks the arguments, fills `a` and launches the streaming kernel (every entry point's first
// launch); the caller launches what sums the split tiles.
static int lin_launch_main(const void* x, int M, int K, int count, const void* const* weights, void* const* outs,
                           const int* Ns, void* workspace, int workgroups, int swiglu, int dtype, hipStream_t st,
                           LinArgs& a) {
  if (!x || !weights || !outs || !Ns) return fail(DLLM_EINVAL, "decode linear: null pointer");
  if (count < 1 || count > LIN_MAXSEG) return fail(DLLM_EINVAL, "decode linear: %d projections (1..%d)", count, LIN_MAXSEG);
  if (M <= 0 || K <= 0 || workgroups <= 0) return fail(DLLM_EINVAL, "decode linear: bad sizes M=%d K=%d", M, K);
  if (dtype != DT_BF16) return fail(DLLM_EUNSUPPORTED, "decode linear: bf16 only");
  if (K % 64) return fail(DLLM_EUNSUPPORTED, "decode linear: K=%d is not a multiple of 64", K);
  if (M > 64) return fail(DLLM_EUNSUPPORTED, "decode linear: M=%d > 64 rows (use a library GEMM)", M);
  if ((uintptr_t)x & 15) return fail(DLLM_EINVAL, "decode linear: x must be 16-byte aligned");
  if (swiglu && (count != 2 || Ns[0] != Ns[1])) return fail(DLLM_EINVAL, "decode linear: swiglu takes gate | up of equal N");
  if (!workspace || ((uintptr_t)workspace & 15)) return fail(DLLM_EINVAL, "decode linear: the workspace must be a 16-byte aligned buffer");
  a = LinArgs{};
  a.x = (const bf16*)x;
  a.nseg = count;
  a.M = M; a.K = K;
  a.ns = K / 64;
  a.swiglu = swiglu;
  long long ntn = 0;
  for (int i = 0; i < count; ++i) {
    if (!weights[i] || !outs[i] || Ns[i] <= 0) return fail(DLLM_EINVAL, "decode linear: projection %d is empty", i);
    if ((uintptr_t)weights[i] & 15) return fail(DLLM_EINVAL, "decode linear: weights must be 16-byte aligned");
    LinSeg& sg = a.seg[i];
    sg.w = (const bf16*)weights[i];
    sg.y = (bf16*)outs[i];
    sg.N = Ns[i];
    sg.tile0 = (int)ntn;
    ntn += (Ns[i] + 127) / 128;
  }
  const long long units = lin_units(M, ntn, K);
  if (units > 0x7fffffffLL) return fail(DLLM_EUNSUPPORTED, "decode linear: %lld work units is too many", units);
  a.ntn = (int)ntn;
  a.units = (int)units;
  a.G = workgroups < units ? workgroups : (int)units;  // no workgroup without units
  if (a.G > 32768) return fail(DLLM_EINVAL, "decode linear: %d workgroups (at most 32768)", workgroups);
  a.uq = a.units / a.G;
  a.ur = a.units % a.G;
  a.part = (float*)workspace;
  a.up = swiglu ? (bf16*)((char*)workspace + (long long)a.G * 2 * LIN_TILE * sizeof(float)) : nullptr;
  decode_linear_kernel<<<dim3((unsigned)a.G), 256, 0, st>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "decode linear launch: %s", hipGetErrorString(e));
  return DLLM_OK;
}

extern "C" int dllm_decode_linear_multi_fwd(const void* x, int M, int K, int count, const void* const* weights,
                                            void* const* outs, const int* Ns, void* workspace, int workgroups,
                                            int swiglu, int dtype, void* stream) {
  LinArgs a;
  hipStream_t st = (hipStream_t)stream;
  const int rc = lin_launch_main(x, M, K, count, weights, outs, Ns, workspace, workgroups, swiglu, dtype, st, a);
  if (rc != DLLM_OK) return rc;
  hipError_t e = hipSuccess;
  if (swiglu) {
    decode_linear_swiglu_kernel<<<dim3((unsigned)(a.seg[1].tile0 * ((M + 31) / 32)), LIN_FIX_CHUNKS), 256, 0, st>>>(a);
  } else {
    // the tiles a range boundary falls inside, in batches of LIN_FIXMAX
    LinFix f;
    f.n = 0;
    for (int b = 1; b <= a.G; ++b) {
      const int ub = b < a.G ? (int)((long long)b * a.units / a.G) : -1;
      const bool split = b < a.G && ub % a.ns != 0;
      if (split && (f.n == 0 || f.tile[f.n - 1] != ub / a.ns)) f.tile[f.n++] = ub / a.ns;
      if (f.n == LIN_FIXMAX || (b == a.G && f.n > 0)) {
        decode_linear_fixup_kernel<<<dim3((unsigned)f.n, LIN_FIX_CHUNKS), 256, 0, st>>>(a, f);
        e = hipGetLastError();
        if (e != hipSuccess) break;
        f.n = 0;
      }
    }
  }
  e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "decode linear fixup launch: %s", hipGetErrorString(e));
  return DLLM_OK;
}

extern "C" int dllm_decode_linear_rmsnorm_fwd(const void* x, const void* weight, void* workspace, int M, int N, int K,
                                              int workgroups, const void* residual, void* sum_out,
                                              const void* norm_weight, void* y, float eps, int unit_offset, int dtype,
                                              int dtype_w, void* stream) {
  if (!residual || !sum_out || !norm_weight || !y) return fail(DLLM_EINVAL, "decode linear rmsnorm: null pointer");
  if (dtype_w != DT_BF16 && dtype_w != DT_F32)
    return fail(DLLM_EUNSUPPORTED, "decode linear rmsnorm: norm weight dtype %d (bf16 or fp32)", dtype_w);
  // up to 8192: the widths the row RMSNorm kernel's vector layout covers (the row of rounded
  // values in LDS is then at most 16 KB)
  if (N <= 0 || N % 512 || N > 8192)
    return fail(DLLM_EUNSUPPORTED, "decode linear rmsnorm: N=%d is not a multiple of 512 up to 8192", N);
  if (((uintptr_t)residual | (uintptr_t)sum_out | (uintptr_t)norm_weight | (uintptr_t)y) & 15)
    return fail(DLLM_EINVAL, "decode linear rmsnorm: residual, sum_out, norm weight and y must be 16-byte aligned");
  if (M <= 0 || workgroups <= 0) return fail(DLLM_EINVAL, "decode linear rmsnorm: bad sizes M=%d workgroups=%d", M, workgroups);
  // the row layout of the row RMSNorm kernel: nw waves (the most, up to 8, dividing N / 512)
  const int nv = N / 512;
  int nw = 8;
  while (nv % nw) --nw;
  const int nvw = nv / nw;
  if (nvw > 8) return fail(DLLM_EUNSUPPORTED, "decode linear rmsnorm: N=%d needs %d vectors per lane (at most 8)", N, nvw);
  // the projection's whole tiles, rounded, go to the workspace after the pieces (the size of
  // dllm_decode_linear_workspace_bytes(M, N, workgroups, 1))
  void* proj = (char*)workspace + (long long)workgroups * 2 * LIN_TILE * sizeof(float);
  const void* w[1] = {weight};
  void* o[1] = {proj};
  const int n[1] = {N};
  LinArgs a;
  hipStream_t st = (hipStream_t)stream;
  const int rc = lin_launch_main(x, M, K, 1, w, o, n, workspace, workgroups, 0, dtype, st, a);
  if (rc != DLLM_OK) return rc;
  // one thread per 4-feature slot (at most 1024, at least the norm's waves)
  const int threads = std::min(1024, std::max(64 * nw, (N / 4 + 63) / 64 * 64));
  const dim3 grid((unsigned)M), block((unsigned)threads);
  const size_t lds = (size_t)N * sizeof(bf16) + 8 * sizeof(float);
  const bf16* r = (const bf16*)residual;
  bf16* so = (bf16*)sum_out;
  bf16* yo = (bf16*)y;
  switch (nvw) {
#define DLLM_LIN_RMS_CASE(NV)                                                                                     \
  case NV:                                                                                                        \
    if (dtype_w == DT_BF16)                                                                                       \
      decode_linear_rmsnorm_kernel<bf16, NV><<<grid, block, lds, st>>>(a, r, so, (const bf16*)norm_weight, yo, eps, \
                                                                      unit_offset, nw);                           \
    else                                                                                                          \
      decode_linear_rmsnorm_kernel<float, NV><<<grid, block, lds, st>>>(a, r, so, (const float*)norm_weight, yo,   \
                                                                       eps, unit_offset, nw);                     \
    break;
    DLLM_LIN_RMS_CASE(1) DLLM_LIN_RMS_CASE(2) DLLM_LIN_RMS_CASE(3) DLLM_LIN_RMS_CASE(4) DLLM_LIN_RMS_CASE(5)
    DLLM_LIN_RMS_CASE(6) DLLM_LIN_RMS_CASE(7) DLLM_LIN_RMS_CASE(8)
#undef DLLM_LIN_RMS_CASE
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "decode linear rmsnorm launch: %s", hipGetErrorString(e));
  return DLLM_OK;
}

extern "C" int dllm_decode_gdn_prologue_fwd(const void* x, int M, int K, const void* const* weights, void* const* outs,
                                            const int* Ns, void* workspace, int workgroups, int T,
                                            const void* conv_prefix, int prefix_len, const void* conv_w,
                                            const void* conv_b, int width, void* mixed, const void* a_log,
                                            const void* dt_bias, float* beta, float* g, int dtype,
                                            int dtype_conv, int dtype_param, void* stream) {
  if (!weights || !outs || !Ns || !conv_w || !mixed || !a_log || !dt_bias || !beta || !g)
    return fail(DLLM_EINVAL, "gdn prologue: null pointer");
  if (T <= 0 || 32 % T || M <= 0 || M % T)
    return fail(DLLM_EUNSUPPORTED, "gdn prologue: T=%d must divide 32 and M=%d", T, M);
  if (width < 2 || width > 4) return fail(DLLM_EUNSUPPORTED, "gdn prologue: conv width %d (2..4)", width);
  if (!(prefix_len == 0 || prefix_len == width - 1) || (prefix_len > 0 && !conv_prefix))
    return fail(DLLM_EINVAL, "gdn prologue: carry-in of %d positions (0 or width - 1 = %d, with a pointer)",
                prefix_len, width - 1);
  if (Ns[2] != Ns[3]) return fail(DLLM_EINVAL, "gdn prologue: b and a of %d and %d heads", Ns[2], Ns[3]);
  if (dtype_conv != DT_BF16 && dtype_conv != DT_F32)
    return fail(DLLM_EUNSUPPORTED, "gdn prologue: conv weight dtype %d", dtype_conv);
  if (dtype_param != DT_BF16 && dtype_param != DT_F32)
    return fail(DLLM_EUNSUPPORTED, "gdn prologue: A_log / dt_bias dtype %d", dtype_param);
  LinArgs a;
  hipStream_t st = (hipStream_t)stream;
  const int rc = lin_launch_main(x, M, K, 4, weights, outs, Ns, workspace, workgroups, 0, dtype, st, a);
  if (rc != DLLM_OK) return rc;
  GdnPrologue p;
  p.prefix = prefix_len > 0 ? (const bf16*)conv_prefix : nullptr;
  p.conv_w = conv_w;
  p.conv_b = conv_b;
  p.mixed = (bf16*)mixed;
  p.a_log = a_log;
  p.dt_bias = dt_bias;
  p.beta = beta;
  p.g = g;
  p.T = T;
  p.width = width;
  p.P = prefix_len;
  const dim3 grid((unsigned)(a.ntn * ((M + 31) / 32)));
  auto go = [&](auto tw, auto tp) {
    using TW = decltype(tw);
    using TP = decltype(tp);
    switch (width) {
      case 2: decode_gdn_prologue_kernel<TW, TP, 2><<<grid, 256, 0, st>>>(a, p); break;
      case 3: decode_gdn_prologue_kernel<TW, TP, 3><<<grid, 256, 0, st>>>(a, p); break;
      default: decode_gdn_prologue_kernel<TW, TP, 4><<<grid, 256, 0, st>>>(a, p); break;
    }
  };
  if (dtype_conv == DT_BF16 && dtype_param == DT_F32) go(bf16{}, float{});
  else if (dtype_conv == DT_BF16) go(bf16{}, bf16{});
  else if (dtype_param == DT_F32) go(float{}, float{});
  else go(float{}, bf16{});
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "gdn prologue launch: %s", hipGetErrorString(e));
  return DLLM_OK;
}

extern "C" int dllm_decode_linear_fwd(const void* x, const void* weight, void* y, void* workspace, int M, int N, int K,
                                      int workgroups, int dtype, void* stream) {
  const void* w[1] = {weight};
  void* o[1] = {y};
  const int n[1] = {N};
  return dllm_decode_linear_multi_fwd(x, M, K, 1, w, o, n, workspace, workgroups, 0, dtype, stream);
}

// ---- allocation-free variant: the split-tile pieces live in a fixed per-device array ----------
//
// For callers that cannot allocate device memory (code under HIP graph capture, serving loops
// that forbid it). The pieces a launch needs are G x 2 x 16 KB (two per workgroup), so the array
// holds 8 MiB = 256 workgroups (one per CU, what dllm_decode_linear_workgroups returns for every
// projection that splits tiles). Every piece the fixup reads is written by the main kernel of the
// same call before it on the same stream, so nothing needs clearing; calls that overlap on one
// GPU (two streams at once) share the array and race.
namespace dllm {
constexpr long long LIN_SCRATCH_BYTES = 8LL << 20;
static __device__ __align__(256) unsigned char scratch[LIN_SCRATCH_BYTES];
constexpr int LIN_MAX_DEVICES = 64;
static void* g_scratch_addr[LIN_MAX_DEVICES];  // device address of `scratch` per device, looked up once
static std::mutex g_scratch_mu;

// Device address of the array on the current device (which must own `stream`).
static int scratch_address(void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(DLLM_ELAUNCH, "decode linear (no-alloc): hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= LIN_MAX_DEVICES) return fail(DLLM_EUNSUPPORTED, "decode linear (no-alloc): device %d", dev);
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    if (e != hipSuccess) return fail(DLLM_EINVAL, "decode linear (no-alloc): hipStreamGetDevice: %s", hipGetErrorString(e));
    if (sdev != dev)
      return fail(DLLM_EINVAL, "decode linear (no-alloc): the stream belongs to device %d, the current device is %d",
                  (int)sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(DLLM_ELAUNCH, "decode linear (no-alloc): hipGetSymbolAddress: %s", hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return DLLM_OK;
}
}  // namespace dllm

extern "C" long long dllm_decode_linear_noalloc_max_bytes(void) { return LIN_SCRATCH_BYTES; }

extern "C" int dllm_decode_linear_fwd_noalloc(const void* x, const void* weight, void* y, int M, int N, int K,
                                              int workgroups, int dtype, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0 || workgroups <= 0)
    return fail(DLLM_EINVAL, "decode linear (no-alloc): bad sizes M=%d N=%d K=%d workgroups=%d", M, N, K, workgroups);
  if (K % 64) return fail(DLLM_EUNSUPPORTED, "decode linear (no-alloc): K=%d is not a multiple of 64", K);
  // the pieces this launch writes: none when every workgroup's unit range is whole tiles
  const long long units = lin_units(M, (N + 127) / 128, K);
  if (units > 0x7fffffffLL) return fail(DLLM_EUNSUPPORTED, "decode linear (no-alloc): %lld work units is too many", units);
  const long long G = workgroups < units ? workgroups : units;
  const long long ns = K / 64;
  bool split = false;
  for (long long b = 1; b < G && !split; ++b) split = (b * units / G) % ns != 0;
  const long long need = split ? G * 2 * LIN_TILE * (long long)sizeof(float) : 0;
  if (need > LIN_SCRATCH_BYTES)
    return fail(DLLM_EUNSUPPORTED,
                "decode linear (no-alloc): %lld workgroups splitting tiles need %lld bytes of scratch, more than the "
                "%lld-byte array (at most %lld such workgroups)", G, need, LIN_SCRATCH_BYTES,
                LIN_SCRATCH_BYTES / (2 * LIN_TILE * (long long)sizeof(float)));
  void* ws = nullptr;
  const int rc = scratch_address(stream, &ws);
  if (rc != DLLM_OK) return rc;
  return dllm_decode_linear_fwd(x, weight, y, ws, M, N, K, workgroups, dtype, stream);
}
