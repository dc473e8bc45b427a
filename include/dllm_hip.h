/*
 * dllm_hip.h — C ABI of the MI355X (gfx950) block-diffusion forward hot path.
 *
 * Conventions (every entry point):
 *  - Tensor arguments are DEVICE pointers owned by the caller; sizes are plain ints; strides are
 *    int64 element counts passed through small HOST arrays.
 *  - `stream` is a hipStream_t (passed as void*); work is enqueued asynchronously on it and the
 *    call never synchronises the device.
 *  - dtype codes: 0 = float32, 1 = bfloat16.
 *  - Return 0 on success or a negative status (-1 invalid argument, -2 unsupported shape/dtype,
 *    -3 launch failure); dllm_last_error() then holds a message (thread-local).
 *  - No entry point allocates device memory; outputs and intermediates are caller buffers.
 *
 * Citations name the reference (kotoba-lang/dllm-qwen38) interface each entry point replaces;
 * [hf] = transformers/models/qwen3_5/modeling_qwen3_5.py (5.15.0).
 */
#ifndef DLLM_HIP_H
#define DLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version of this header/library pair. */
int dllm_abi_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char* dllm_last_error(void);

/*
 * Chunked gated delta rule with per-chunk states.
 * Replaces src/dllm_qwen38/gdn.py:48-123 chunk_gated_delta_rule_with_states (and the core
 * dispatch gdn.py:147-163 _core). q/k [B,T,Hk,Dk], v [B,T,Hv,Dv] with arbitrary batch/token/head
 * strides (last dim contiguous); Hk divides Hv and value head j reads key head j/(Hv/Hk), so
 * already-expanded q/k (Hk == Hv) are accepted as the reference passes them. g and beta
 * [B,T,Hv] fp32 (the reference casts both to fp32, gdn.py:76-79). initial_state [B,Hv,Dk,Dv] fp32 or NULL (zeros).
 * out [B,T,Hv,Dv] contiguous in the input dtype. states [B,T/chunk,Hv,Dk,Dv] fp32 (state after
 * each chunk) or NULL for need_states=False. scale multiplies q after the optional l2norm
 * (the reference uses Dk^-1/2). T % chunk != 0 fails with the reference's ValueError text.
 * Dk, Dv <= 128.
 */
int dllm_gdn_chunk_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                       const void* v, const int64_t* v_strides, const float* g, const int64_t* g_strides,
                       const float* beta, const int64_t* beta_strides, const float* initial_state,
                       void* out, float* states, int B, int T, int Hk, int Hv, int Dk, int Dv,
                       int chunk, int dtype, int use_qk_l2norm, float scale, void* stream);

/*
 * 1 if the fused state-fork kernel handles (Dk, block, dtype): block divides 32, Dk <= 128, and
 * Dk <= 64 for float32. Otherwise callers run the two-pass fork (dllm_gdn_chunk_fwd on the clean
 * stream with states, then again on the B*nb noised rows with initial states), as the reference
 * does at src/dllm_qwen38/blockdiff.py:160-176.
 */
int dllm_gdn_fused_fork_supported(int Dk, int block, int dtype);

/*
 * Which kernel dllm_gdn_state_fork_fwd runs for (Dk, Dv, block, dtype) on 16-byte aligned
 * activations: 2 = the pipelined fork kernel (bf16 heads of 128 x 128), 1 = the first fused fork
 * kernel (other shapes dllm_gdn_fused_fork_supported accepts), 0 = neither (the caller runs the
 * two-pass fork). The reference reports the core it ran through last_impl()
 * (src/dllm_qwen38/gdn.py:44-45); this is the same report one level down.
 */
int dllm_gdn_state_fork_path(int Dk, int Dv, int block, int dtype);

/*
 * Fused state fork of one GDN layer, both streams in one launch.
 * Replaces the LINEAR arm of src/dllm_qwen38/blockdiff.py:153-177 (the clean pass
 * gdn_mixer_forward(need_states=True) at :160, the state shift at :165-166 and the relaunch of
 * every noised block as a batch row at :174-176), core part (gdn.py:221-231).
 * qkv0/qkvt: post-conv activations [B,L,conv_dim] (strides in elements; channels contiguous)
 * laid out as q | k | v channel blocks of Hk*Dk, Hk*Dk and Hv*Dv (gdn.py:221-224).
 * beta* and g* [B,L,Hv] fp32, contiguous.
 * out0/outt [B,L,Hv,Dv] contiguous: clean output, and noised output where noised block k of
 * sequence b starts from the clean state after block k-1 (zeros for k = 0).
 * states [B,L/block,Hv,Dk,Dv] fp32 (clean state after every block) or NULL.
 */
int dllm_gdn_state_fork_fwd(const void* qkv0, const void* qkvt, int64_t qkv_stride_b, int64_t qkv_stride_t,
                            const float* beta0, const float* betat, const float* g0, const float* gt,
                            void* out0, void* outt, float* states, int B, int L, int Hk, int Hv, int Dk,
                            int Dv, int block, int dtype, float scale, void* stream);

/*
 * The same op over blocks [block_begin, block_end) of every sequence, for callers that overlap the
 * conv of later blocks with the fork of earlier ones (the reference has no such split: it is the
 * blockdiff.py:153-177 arm above, cut along the sequence). All pointers and sizes are those of the
 * whole op; outputs and states are written for the range only. A range after block 0 starts from
 * the clean state after block block_begin - 1, read from states (which must not be NULL and must
 * hold that snapshot, as the range before it writes). Ranges run the pipelined fork kernel only
 * (dllm_gdn_state_fork_path() == 2); other shapes return -2 (unsupported) unless the range is the
 * whole sequence. Running consecutive ranges in order gives the whole op's results bit for bit.
 */
int dllm_gdn_state_fork_range_fwd(const void* qkv0, const void* qkvt, int64_t qkv_stride_b,
                                  int64_t qkv_stride_t, const float* beta0, const float* betat,
                                  const float* g0, const float* gt, void* out0, void* outt, float* states,
                                  int B, int L, int Hk, int Hv, int Dk, int Dv, int block, int dtype,
                                  float scale, int block_begin, int block_end, void* stream);

/*
 * Bounded waits inside kernels (the pipelined fork's LDS row-buffer hand-off between its waves)
 * give up after a limit and set a bit in a per-device status word instead of hanging:
 * 1 = LDS row-buffer wait; a launch that set a bit produced invalid outputs.
 * dllm_status synchronises the device and returns the bits of the current device (>= 0; reset != 0
 * clears them). dllm_set_spin_limit sets the limit in sleeps (default 1 << 20, about 30-60 ms per
 * wait; process-wide) and returns the previous one; tests lower it to exercise the reporting. No
 * counterpart in the reference, whose CPU path has no such waits.
 */
int dllm_status(int reset);
int dllm_set_spin_limit(int limit);
/*
 * The pipelined fork splits each head's value columns over two workgroups when twice the
 * (sequence, value head) count fits the device's compute units (mode 0, the default); mode 1
 * never splits, mode 2 always does. Results are identical either way. Process-wide; returns the
 * previous mode. For tests and measurement; no counterpart in the reference.
 */
/*
 * dllm_gdn_state_fork_range_fwd with the v channels' short conv done inside the fork kernel. The
 * reference runs the conv of all channels first (src/dllm_qwen38/gdn.py:217-219 with the noised
 * prefix cut at blockdiff.py:167-173) and then the core; here the conv launch
 * (dllm_conv_fork_channels_range_fwd with y_channels = 2*Hk*Dk) writes only the q and k channels,
 * and the fork reads the v channels' pre-conv rows and convolves them (width 4 + SiLU, the
 * dllm_conv_fork_fwd arithmetic, bit for bit), which saves the v channels' round trip through HBM.
 * qk0/qkt: the conv outputs (q and k channels read); raw0/rawt: the conv inputs (v channels read),
 * both [B,L,conv_dim] with the strides given. conv_weight [conv_dim,4] bf16 or fp32 (dtype_w),
 * conv_bias [conv_dim] of that dtype or NULL. conv_tails: the [B*nb,conv_dim,3] tails tensor,
 * whose v channels this call writes for its blocks (4-byte aligned, conv_dim even), or NULL.
 * The pipelined fork kernel only (dllm_gdn_state_fork_path() == 2; else -2). No fault flags.
 */
int dllm_gdn_state_fork_vconv_range_fwd(const void* qk0, const void* qkt, const void* raw0, const void* rawt,
                                        int64_t stride_b, int64_t stride_t, const void* conv_weight,
                                        const void* conv_bias, int dtype_w, void* conv_tails, int conv_dim,
                                        const float* beta0, const float* betat, const float* g0,
                                        const float* gt, void* out0, void* outt, float* states, int B, int L,
                                        int Hk, int Hv, int Dk, int Dv, int block, int dtype, float scale,
                                        int block_begin, int block_end, void* stream);

int dllm_set_fork_split(int mode);
/* Test only: with on != 0, the LDS row-buffer wait waits for a count that is never reached, so
 * every such wait gives up after the spin limit (the kernel still ends, outputs invalid). Returns
 * the previous mode. */
int dllm_set_wait_test_mode(int on);

/*
 * Causal depthwise conv + SiLU of both fork streams with conv-prefix carry-in.
 * Replaces [hf]:219-239 causal_conv1d_fn as called at src/dllm_qwen38/gdn.py:217-219 for the clean
 * stream and for the noised rows with the prefix cut at src/dllm_qwen38/blockdiff.py:167-173.
 * raw0/rawt [B,L,conv_dim] token-major contiguous; weight [conv_dim,width] (+ optional bias).
 * y0/yt [B,L,conv_dim] (input dtype). tails [B*nb,conv_dim,width-1] (input dtype) receives the
 * clean pre-conv values before every block (zeros before the sequence start), or NULL.
 * flags bit 0: the "no-conv-prefix" fault (noised blocks start cold, blockdiff.py:88,168-169).
 * Computes in the weight dtype (fp32 accumulate, rounded to it), returns the input dtype.
 */
int dllm_conv_fork_fwd(const void* raw0, const void* rawt, const void* weight, const void* bias,
                       void* y0, void* yt, void* tails, int B, int L, int conv_dim, int width,
                       int block, int dtype_x, int dtype_w, int flags, void* stream);

/*
 * dllm_conv_fork_fwd over blocks [block_begin, block_end) of every sequence (rows, tails and the
 * prefix carry-in of those blocks; the carry-in reads the rows before block_begin). The split that
 * dllm_gdn_state_fork_range_fwd takes, for the same overlap; no counterpart in the reference.
 */
int dllm_conv_fork_range_fwd(const void* raw0, const void* rawt, const void* weight, const void* bias,
                             void* y0, void* yt, void* tails, int B, int L, int conv_dim, int width,
                             int block, int dtype_x, int dtype_w, int flags, int block_begin,
                             int block_end, void* stream);

/*
 * dllm_conv_fork_range_fwd over channels [0, y_channels) only (their y rows and tails; the other
 * channels of y0, yt and tails are left untouched). For dllm_gdn_state_fork_vconv_range_fwd, which
 * convolves the v channels itself; no counterpart in the reference. 0 <= y_channels <= conv_dim.
 */
int dllm_conv_fork_channels_range_fwd(const void* raw0, const void* rawt, const void* weight, const void* bias,
                                      void* y0, void* yt, void* tails, int B, int L, int conv_dim, int width,
                                      int block, int dtype_x, int dtype_w, int flags, int block_begin,
                                      int block_end, int y_channels, void* stream);

/*
 * Generic causal depthwise conv (+ optional SiLU) with an optional prefix.
 * Replaces [hf]:219-239 causal_conv1d_fn on cat([conv_prefix, x]) keeping the last T outputs
 * (src/dllm_qwen38/gdn.py:217-219). x [B,C,T] with strides {b,c,t}; prefix [B,C,prefix_len] with
 * strides or NULL; weight [C,width], width <= 8. y is written token-major [B,T,C] contiguous.
 */
int dllm_causal_conv1d_fwd(const void* x, const int64_t* x_strides, const void* prefix,
                           const int64_t* prefix_strides, int prefix_len, const void* weight,
                           const void* bias, void* y, int B, int C, int T, int width, int dtype_x,
                           int dtype_w, int activation, void* stream);

/*
 * Integer fork layout, computed on the device with the same index functions the kernels use.
 * Replaces the index arithmetic of src/dllm_qwen38/blockdiff.py:161-173:
 *   row[b*nb+k]          = fork batch row of (sequence b, block k)            (int32 [B*nb])
 *   state_src[row]       = flat clean-state index b*nb+k-1 the row starts from, -1 = zeros
 *   prefix_pos[row*(width-1)+j] = clean position feeding conv-prefix slot j, -1 = zero pad
 */
int dllm_fork_layout(int B, int L, int block, int width, int32_t* row, int32_t* state_src,
                     int32_t* prefix_pos, void* stream);

/*
 * Complementary-mask block-diffusion attention (flash style, hidden tiles skipped).
 * Replaces the FULL arm of src/dllm_qwen38/blockdiff.py:178-182 with the [2L,2L] additive mask of
 * blockdiff.py:50-66 (never materialised here) and [hf]:604-626 eager_attention_forward (GQA by
 * indexing instead of repeat_kv). q [B,2L,Hq,d], k/v [B,2L,Hkv,d] (halves ordered
 * cat([x_t, x_0]), rotary already applied), strides {b,t,h} in elements, last dim contiguous;
 * out [B,2L,Hq,d] contiguous, same dtype. Visibility with blocks of `block` tokens per half:
 * x_t->x_t same block, x_t->x_0 earlier blocks, x_0->x_0 block-causal, x_0->x_t never.
 * flags bit 0: the "mask-leak" fault (x_t block k also sees x_t blocks < k, blockdiff.py:61).
 * Scores and softmax in fp32; P rounded to the input dtype before P.V ([hf]:621-622); d <= 256.
 */
int dllm_bd_attention_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                          const void* v, const int64_t* v_strides, void* out, int B, int L, int Hq, int Hkv,
                          int d, int block, float scale, int dtype, int flags, void* stream);

/*
 * The gated attention layer's core in one launch: dllm_bd_attention_fwd with the q prologue and the
 * output gate fused in. Replaces, of Qwen3_5Attention.forward ([hf]:656-701, called from
 * src/dllm_qwen38/blockdiff.py:178-182), the q RMSNorm(1 + w) ([hf]:672), the partial RoPE of q
 * ([hf]:676, apply_rotary_pos_emb [hf]:554-589), the attention ([hf]:682-695) and the sigmoid
 * output gate ([hf]:698); k arrives already normed and rotated (dllm_qk_norm_rope_fwd with Hq = 0),
 * v as projected. q_norm_w non-null: q [B,2L,Hq,d] is the raw q_proj query half (any strides, last
 * dim contiguous); each row is normalised with q_norm_w (q_norm_dtype 0 fp32 / 1 bf16) and q_norm_eps
 * and its first rotary_dim dims rotated with the [L, rotary_dim] cos/sin tables (activation dtype)
 * at the row's position within its half, rounded as dllm_qk_norm_rope_fwd rounds. q_norm_w null: q
 * is used as given. gate non-null: out = bf16(bf16(attention) * bf16(sigmoid(gate))) with gate
 * [B,2L,Hq,d] at gate_strides (the q_proj gate half). bf16, d in {64, 128, 256}, rotary_dim a
 * multiple of 64 (dllm_bd_attention_gated_supported), 16-byte aligned q/k/v rows, norm weight and
 * tables; anything else returns -2 (the caller runs the separate launches).
 */
int dllm_bd_attention_gated_supported(int d, int rotary_dim, int dtype);
int dllm_bd_attention_gated_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                                const void* v, const int64_t* v_strides, const void* gate,
                                const int64_t* gate_strides, const void* q_norm_w, int q_norm_dtype,
                                float q_norm_eps, const void* cos_table, const void* sin_table, int rotary_dim,
                                void* out, int B, int L, int Hq, int Hkv, int d, int block, float scale, int dtype,
                                int flags, void* stream);

/*
 * Block-causal attention of a query segment against a key/value cache: the clean-prefix cache of a
 * cached decoder. The reference decoder (src/dllm_qwen38/decode.py:63-66) re-runs the whole
 * two-stream forward per denoising step; there, x_t block k sees x_0 blocks < k and itself
 * (blockdiff.py:50-66), and the clean stream is block-causal (blockdiff.py:43-47). With the clean
 * prefix's K/V kept, one step is this call with the block's queries. q [B,M,Hq,d] at absolute
 * positions q0..q0+M-1; k/v [B,N,Hkv,d] at positions 0..N-1 (rotary already applied); query i sees
 * key j iff j/block <= (q0+i)/block. A denoising step is M = block, q0 = N - block (every key
 * visible); a prompt prefill is q0 = 0, M = N. Strides {b,t,h} in elements, last dim contiguous;
 * out [B,M,Hq,d] contiguous, same dtype. Same numerics as dllm_bd_attention_fwd; d <= 256.
 * key_splits > 1 (bf16, d in {64,128,256}; a decoding step's few query rows against a long cache):
 * the key tiles are split over that many workgroups per query tile and head, and a second launch
 * merges their partial results (flash-decoding); workspace then holds key_splits*B*M*Hq*(d+2)
 * floats. Other shapes ignore key_splits.
 */
int dllm_block_causal_attention_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                                    const void* v, const int64_t* v_strides, void* out, int B, int M, int N, int q0,
                                    int Hq, int Hkv, int d, int block, float scale, int dtype, float* workspace,
                                    int key_splits, void* stream);

/*
 * The same with the gated attention layer's output gate ([hf]:698, o * sigmoid(gate) before o_proj,
 * as the cached decoder's attention layer runs it) applied at the output store or the merge of the
 * key shares: out = bf16(bf16(attention) * bf16(sigmoid(gate))), the rounding of the separate
 * elementwise product. gate [B,M,Hq,d] bf16 with strides {b,t,h} in elements (multiples of 4,
 * 8-byte aligned rows; the gate half of the q_proj output read in place). Takes the direct-load
 * kernel's shapes only (bf16, d in {64,128,256}, 16-byte aligned q/k/v rows, positive scale);
 * others return -2.
 */
int dllm_block_causal_attention_gated_fwd(const void* q, const int64_t* q_strides, const void* k,
                                          const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                          const void* gate, const int64_t* gate_strides, void* out, int B, int M,
                                          int N, int q0, int Hq, int Hkv, int d, int block, float scale, int dtype,
                                          float* workspace, int key_splits, void* stream);

/*
 * Projections of a decoding step (few token rows): y[M,N] = x[M,K] W[N,K]^T, bf16 in and out, fp32
 * accumulation; M <= 64, K a multiple of 64, x and W row-major and 16-byte aligned, y [M,N]
 * contiguous. Replaces the nn.Linear calls (in_proj_*, q/k/v/o_proj, the MLP, lm_head) that every
 * denoising step of the reference decoder runs inside block_diffusion_forward
 * (src/dllm_qwen38/decode.py:63-66; [hf]:168-184,656-717) when they see one block of tokens.
 * The launch has `workgroups` workgroups (at most 32768), each streaming an equal share of the
 * (128-feature x 32-row tile, 64-k step) units; dllm_decode_linear_workgroups(M, N, K) gives one per
 * CU, or one per tile when there are at least two tiles per CU (0 if the shape is not taken). Tiles
 * split between workgroups leave fp32 pieces in `workspace` (dllm_decode_linear_workspace_bytes
 * bytes, 16-byte aligned), which a second launch sums in workgroup order: deterministic for a given
 * workgroup count.
 */
int dllm_decode_linear_workgroups(int M, int N, int K);
long long dllm_decode_linear_workspace_bytes(int M, int N_gate, int workgroups, int swiglu);
int dllm_decode_linear_fwd(const void* x, const void* weight, void* y, void* workspace, int M, int N, int K,
                           int workgroups, int dtype, void* stream);

/*
 * dllm_decode_linear_fwd without a workspace argument: no counterpart in the reference. For callers
 * that cannot allocate device memory (code under HIP graph capture, serving loops that forbid
 * allocation). The split-tile pieces go to a fixed per-device array inside the library of
 * dllm_decode_linear_noalloc_max_bytes() bytes (8 MiB: 256 workgroups that split tiles, one per
 * CU); a launch needing more returns -2 with a message, and one that splits no tile has no limit.
 * Nothing is allocated. The current device must own `stream`. Calls that overlap on one GPU (two
 * streams at once) share the array and race.
 */
long long dllm_decode_linear_noalloc_max_bytes(void);
int dllm_decode_linear_fwd_noalloc(const void* x, const void* weight, void* y, int M, int N, int K, int workgroups,
                                   int dtype, void* stream);

/*
 * Up to four projections of the same x in one launch (q | k | v; in_proj_qkv | z | b | a; gate |
 * up): weights[i] [Ns[i], K] -> outs[i] [M, Ns[i]], one workgroup count for all (from
 * dllm_decode_linear_workgroups(M, sum of Ns rounded up to 128, K)); workspace of
 * dllm_decode_linear_workspace_bytes(M, Ns[0], workgroups, swiglu) bytes. swiglu = 1 (two
 * projections gate | up of equal N): outs[0] receives round(round(silu(gate)) * up), the MLP
 * activation of [hf]:704-717, and outs[1] is not written.
 */
int dllm_decode_linear_multi_fwd(const void* x, int M, int K, int count, const void* const* weights, void* const* outs,
                                 const int* Ns, void* workspace, int workgroups, int swiglu, int dtype, void* stream);

/*
 * The Gated DeltaNet mixer's input projections of a decoding step finished together with what reads
 * them next (src/dllm_qwen38/gdn.py:212-226 with conv_prefix, as the cached decoder runs it):
 * weights[0..3] = in_proj_qkv [C, K], in_proj_z, in_proj_b [H, K], in_proj_a [H, K] into
 * outs[0..3] [M, Ns[i]] (bf16, contiguous), one launch as dllm_decode_linear_multi_fwd (same
 * workgroups and workspace), then one launch that sums the split tiles and forms
 * mixed [M, C] = SiLU(causal depthwise conv of the qkv projection, width 2..4), the history
 * before each sequence's first token taken from conv_prefix [M/T, C, width-1] (prefix_len =
 * width - 1; prefix_len = 0: zeros), beta [M, H] = sigmoid(b) rounded to bf16 and
 * g [M, H] = -exp(A_log) softplus(a + dt_bias) (fp32). Rows are M/T sequences of T tokens, T
 * dividing 32. Element for element the results of dllm_decode_linear_multi_fwd,
 * dllm_causal_conv1d_fwd (activation on) and dllm_gdn_gates_fwd run separately. conv_w [C, width]
 * and conv_b [C] (nullable) in dtype_conv, A_log and dt_bias [H] in dtype_param (bf16 or fp32).
 */
int dllm_decode_gdn_prologue_fwd(const void* x, int M, int K, const void* const* weights, void* const* outs,
                                 const int* Ns, void* workspace, int workgroups, int T, const void* conv_prefix,
                                 int prefix_len, const void* conv_w, const void* conv_b, int width, void* mixed,
                                 const void* a_log, const void* dt_bias, float* beta, float* g, int dtype,
                                 int dtype_conv, int dtype_param, void* stream);

/*
 * A projection followed by the residual add and RMSNorm of the next module, as the decoder layer
 * runs them after o_proj / out_proj and after down_proj ([hf]:778-792; the post-attention norm,
 * the next layer's input norm, the final norm): s = round(x W^T) + residual rounded to bf16 (written
 * to sum_out) and y = s * rsqrt(mean(s^2) + eps) * (1 + w) (unit_offset = 1; 0: w as is), equal
 * element for element to dllm_decode_linear_fwd followed by dllm_rmsnorm_fwd(.., residual,
 * sum_out, ..), with the fixup launch of the first and the separate norm folded into one row-wise
 * launch. x [M, K], W [N, K], residual / sum_out / y [M, N] bf16; norm weight [N] bf16 or fp32
 * (dtype_w); N a multiple of 512 up to 8192; workgroups from dllm_decode_linear_workgroups(M, N,
 * K); workspace of dllm_decode_linear_workspace_bytes(M, N, workgroups, 1) bytes (the pieces, then
 * the projection's rounded whole tiles). All pointers 16-byte aligned.
 */
int dllm_decode_linear_rmsnorm_fwd(const void* x, const void* weight, void* workspace, int M, int N, int K,
                                   int workgroups, const void* residual, void* sum_out, const void* norm_weight,
                                   void* y, float eps, int unit_offset, int dtype, int dtype_w, void* stream);

/*
 * Qwen3.5 RMSNorm over the last dim of x [rows, dim]: y = x * rsqrt(mean(x^2) + eps) * (1 + w)
 * in fp32 (unit_offset = 1; 0 applies w as is), rounded once to x's dtype.
 * Replaces [hf]:720-737 Qwen3_5RMSNorm as called by the decoder layer and the final norm
 * (src/dllm_qwen38/blockdiff.py:150,186-187,200). With residual != NULL the normed value is
 * s = x + residual rounded to x's dtype (the residual adds of [hf]:785,791), and s is also written
 * to sum_out when that is non-NULL. All tensors contiguous; weight [dim].
 */
int dllm_rmsnorm_fwd(const void* x, const void* residual, void* sum_out, const void* weight, void* y,
                     int rows, int dim, float eps, int dtype, int dtype_w, int unit_offset, void* stream);

/*
 * Gated RMSNorm of the GDN output: y = round(w * round(rmsnorm(x))) * silu(z), rounded to x's dtype.
 * Replaces [hf]:168-184 Qwen3_5RMSNormGated as called at src/dllm_qwen38/gdn.py:232.
 * x, z [rows, dim] contiguous; weight [dim].
 */
int dllm_gated_rmsnorm_fwd(const void* x, const void* z, const void* weight, void* y, int rows, int dim,
                           float eps, int dtype, int dtype_w, void* stream);

/*
 * Gated DeltaNet gates (src/dllm_qwen38/gdn.py:225-226): beta = sigmoid(b) rounded to the input
 * dtype and held in fp32 (the core's beta), g = -exp(A_log) * softplus(a + dt_bias) in fp32
 * (softplus linear above 20). b, a [rows, heads] contiguous in dtype; A_log, dt_bias [heads] in
 * dtype_param; beta, g [rows, heads] fp32.
 */
int dllm_gdn_gates_fwd(const void* b, const void* a, const void* a_log, const void* dt_bias, float* beta, float* g,
                       int64_t rows, int heads, int dtype, int dtype_param, void* stream);

/*
 * SwiGLU product of the MLP: out = round(round(silu(gate)) * up), n elements, 16-byte aligned.
 * Replaces the act_fn(gate_proj(x)) * up_proj(x) of [hf]:704-717.
 */
int dllm_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream);

/*
 * The same over rows [rows, cols] whose gate and up rows are ld elements apart (the two halves of
 * one fused gate | up projection, [hf]:704-717 with both weights in one GEMM): out contiguous;
 * cols and ld multiples of 8, 16-byte aligned pointers.
 */
int dllm_swiglu_rows_fwd(const void* gate, const void* up, int64_t ld, void* out, int64_t rows, int64_t cols,
                         int dtype, void* stream);

/*
 * Attention prologue: per (token, head) row of q [B,S,Hq,hd] and k [B,S,Hkv,hd] (strides {b,t,h}
 * in elements, last dim contiguous): RMSNorm over hd with (1 + w), then partial RoPE on the first
 * rotary_dim dims, out = a*cos + rotate_half(a)*sin with products and sum rounded to the dtype.
 * Token t reads table row t mod L (positions shared by both halves of cat([x_t, x_0]),
 * src/dllm_qwen38/blockdiff.py:143-144). cos/sin [L, rotary_dim] in the activation dtype.
 * Writes contiguous q_out [B,S,Hq,hd], k_out [B,S,Hkv,hd]. hd <= 256. dtype / dtype_w: bf16 / bf16,
 * bf16 / fp32 (norm weights kept in fp32) or fp32 / fp32. Hq = 0: the k rows alone
 * (q, q_strides, q_norm_w and q_out may be null), for a layer whose q prologue runs inside
 * dllm_bd_attention_gated_fwd.
 * Replaces [hf]:672-680 (q_norm, k_norm, apply_rotary_pos_emb [hf]:554-589).
 */
int dllm_qk_norm_rope_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                          const void* q_norm_w, const void* k_norm_w, const void* cos_table,
                          const void* sin_table, void* q_out, void* k_out, int B, int S, int L, int Hq,
                          int Hkv, int head_dim, int rotary_dim, float eps, int dtype, int dtype_w,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DLLM_HIP_H */
