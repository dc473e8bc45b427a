"""Every C-ABI entry point refuses invalid arguments with the documented status (-1 invalid argument,
-2 unsupported shape or dtype) and a message, before it launches anything: these run on the host
with placeholder device addresses, which no refused call dereferences. The reference's own shape
contracts are among them: `T % chunk` (src/dllm_qwen38/gdn.py:70-71) and `L % block`
(src/dllm_qwen38/blockdiff.py:133-137)."""

import ctypes

import pytest
import torch

from dllm_qwen38_amd import _lib

# The placeholder addresses must never reach a device: should a host-side check regress, the call
# would launch a kernel on an unmapped address. These checks need no GPU, so where a ROCm device is
# visible (a full, unfiltered run on a GPU machine) the module is skipped; the CPU suite runs them.
if torch.cuda.device_count() > 0:
    pytest.skip("host-only refusal checks with placeholder device addresses: skipped where a GPU is visible",
                allow_module_level=True)

EINVAL, EUNSUP = -1, -2
P = 1 << 16            # a 16-byte aligned placeholder address
P2 = P + 2             # a misaligned one
BF, F32 = _lib.DT_BF16, _lib.DT_F32


def s3(*v):
    return (ctypes.c_int64 * 3)(*v)


def ptrs(*v):
    return (ctypes.c_void_p * len(v))(*v)


def ints(*v):
    return (ctypes.c_int * len(v))(*v)


def chunk(q=P, B=1, T=64, Hk=2, Hv=4, Dk=64, Dv=64, chunk=32, dtype=F32, st=(4096, 64, 16)):
    """dllm_gdn_chunk_fwd with [B, T, H, D] tensors of token stride st[1]."""
    return ("dllm_gdn_chunk_fwd", q, s3(*st), P, s3(*st), P, s3(*st), P, s3(*st), P, s3(*st), None, P, None,
            B, T, Hk, Hv, Dk, Dv, chunk, dtype, 1, 0.125, None)


def fork(qkv0=P, B=1, L=64, Hk=2, Hv=2, Dk=128, Dv=128, block=32, dtype=BF, states=P, stride_t=768,
         rng=None):
    """dllm_gdn_state_fork_fwd (or the range entry with rng = (begin, end))."""
    head = (qkv0, P, stride_t * L, stride_t, P, P, P, P, P, P, states, B, L, Hk, Hv, Dk, Dv, block, dtype, 0.088)
    if rng is None:
        return ("dllm_gdn_state_fork_fwd", *head, None)
    return ("dllm_gdn_state_fork_range_fwd", *head, rng[0], rng[1], None)


def conv(raw0=P, B=1, L=64, Cd=64, width=4, block=32, dx=BF, dw=BF, rng=None):
    head = (raw0, P, P, None, P, P, P, B, L, Cd, width, block, dx, dw, 0)
    if rng is None:
        return ("dllm_conv_fork_fwd", *head, None)
    return ("dllm_conv_fork_range_fwd", *head, rng[0], rng[1], None)


def vfork(qk=P, raw=P, w=P, dtw=BF, tails=P, cd=768, B=1, L=64, Hk=2, Hv=2, Dk=128, Dv=128, block=32, dtype=BF,
          stride_t=768):
    """dllm_gdn_state_fork_vconv_range_fwd over the whole sequence."""
    return ("dllm_gdn_state_fork_vconv_range_fwd", qk, P, raw, P, stride_t * L, stride_t, w, None, dtw, tails, cd,
            P, P, P, P, P, P, P, B, L, Hk, Hv, Dk, Dv, block, dtype, 0.088, 0, max(1, L // block), None)


def convc(yc, Cd=64):
    """dllm_conv_fork_channels_range_fwd over blocks [0, 2) with y_channels = yc."""
    return ("dllm_conv_fork_channels_range_fwd", P, P, P, None, P, P, P, 1, 64, Cd, 4, 32, BF, BF, 0, 0, 2, yc, None)


def conv1d(x=P, B=1, C=64, T=16, width=4, prefix=None, plen=0, dx=BF, dw=BF):
    return ("dllm_causal_conv1d_fwd", x, s3(T * C, C, 1), prefix, s3(3 * C, 3, 1) if plen else None, plen, P, None,
            P, B, C, T, width, dx, dw, 1, None)


def bd(q=P, B=1, L=64, Hq=4, Hkv=2, d=64, block=32, dtype=BF, st_t=256):
    return ("dllm_bd_attention_fwd", q, s3(st_t * 2 * L, st_t, d), P, s3(st_t * 2 * L, st_t, d), P,
            s3(st_t * 2 * L, st_t, d), P, B, L, Hq, Hkv, d, block, 0.125, dtype, 0, None)


def gated(q=P, B=1, L=64, Hq=4, Hkv=2, d=256, block=32, dtype=BF, rd=64, qnw=P, gate=P, cos=P, wdt=BF, st_t=1024):
    """dllm_bd_attention_gated_fwd with the q prologue (qnw) and the gate."""
    return ("dllm_bd_attention_gated_fwd", q, s3(st_t * 2 * L, st_t, d), P, s3(st_t * 2 * L, st_t, d), P,
            s3(st_t * 2 * L, st_t, d), gate, s3(st_t * 2 * L, st_t, d) if gate else None, qnw, wdt, 1e-6, cos, P, rd,
            P, B, L, Hq, Hkv, d, block, 0.0625, dtype, 0, None)


def bc(B=1, M=32, N=96, q0=64, Hq=4, Hkv=2, d=64, block=32, ws=None, splits=1):
    return ("dllm_block_causal_attention_fwd", P, s3(M * 256, 256, 64), P, s3(N * 128, 128, 64), P,
            s3(N * 128, 128, 64), P, B, M, N, q0, Hq, Hkv, d, block, 0.125, BF, ws, splits, None)


def rope(q=P, B=1, S=8, L=8, Hq=4, Hkv=2, hd=64, rd=16, cos=P, dt=BF, dtw=BF, qst=(2048, 256, 64), k=P):
    return ("dllm_qk_norm_rope_fwd", q, s3(*qst), k, s3(1024, 128, 64), P, P, cos, P, P, P,
            B, S, L, Hq, Hkv, hd, rd, 1e-6, dt, dtw, None)


def multi(x=P, M=32, K=128, count=1, Ns=(128,), ws=P, wgs=4, swiglu=0, dtype=BF, w=None):
    w = w or (P,) * len(Ns)
    return ("dllm_decode_linear_multi_fwd", x, M, K, count, ptrs(*w), ptrs(*(P,) * len(Ns)), ints(*Ns), ws, wgs,
            swiglu, dtype, None)


def linrms(x=P, M=32, N=512, K=128, wgs=4, r=P, so=P, nw=P, y=P, dtype=BF, dtype_w=BF, ws=P):
    """dllm_decode_linear_rmsnorm_fwd (the projection, then the residual add and RMSNorm)."""
    return ("dllm_decode_linear_rmsnorm_fwd", x, P, ws, M, N, K, wgs, r, so, nw, y, 1e-6, 1, dtype, dtype_w, None)


def prologue(M=32, T=32, Ns=(768, 512, 16, 16), prefix=P, plen=3, width=4, dconv=BF, dparam=F32, mixed=P, K=96):
    """dllm_decode_gdn_prologue_fwd (in_proj_qkv | z | b | a, then the conv and the gates); K = 96 makes
    an argument set that passes the prologue's own checks fail in the projection's."""
    return ("dllm_decode_gdn_prologue_fwd", P, M, K, ptrs(P, P, P, P), ptrs(P, P, P, P), ints(*Ns), P, 4, T, prefix,
            plen, P, None, width, mixed, P, P, P, P, BF, dconv, dparam, None)


CASES = {
    # chunked gated delta rule (src/dllm_qwen38/gdn.py:48-123)
    "chunk null pointer": (chunk(q=None), EINVAL, "gdn: null pointer"),
    "chunk empty batch": (chunk(B=0), EINVAL, "bad sizes"),
    "chunk T % chunk": (chunk(T=100), EINVAL, "sequence_length 100 is not a multiple of chunk_size 32"),
    "chunk GQA ratio": (chunk(Hk=3, Hv=4), EINVAL, "Hv=4 is not a multiple of Hk=3"),
    "chunk Dk > 128": (chunk(Dk=256), EUNSUP, "Dk=256 > 128"),
    "chunk Dv > 128": (chunk(Dv=192), EUNSUP, "Dv=192 > 128"),
    "chunk dtype": (chunk(dtype=7), EUNSUP, "dtype 7 not supported"),
    "chunk 32-bit extent": (chunk(T=1 << 16, st=(1 << 30, 1 << 16, 64)), EUNSUP, "32-bit element offsets"),
    # state fork (src/dllm_qwen38/blockdiff.py:153-177)
    "fork null pointer": (fork(qkv0=None), EINVAL, "gdn fork: null pointer"),
    "fork empty batch": (fork(B=0), EINVAL, "gdn fork: bad sizes"),
    "fork L % block": (fork(L=100), EINVAL, "L=100 is not a multiple of block=32"),
    "fork GQA ratio": (fork(Hk=2, Hv=3), EINVAL, "Hv=3 is not a multiple of Hk=2"),
    "fork block 64": (fork(block=64), EUNSUP, "fused fork unsupported"),
    "fork block 24": (fork(L=96, block=24), EUNSUP, "fused fork unsupported"),
    "fork fp32 Dk 128": (fork(dtype=F32), EUNSUP, "fused fork unsupported"),
    "fork 32-bit extent": (fork(L=1 << 16, stride_t=1 << 16), EUNSUP, "32-bit element offsets"),
    "range empty": (fork(rng=(1, 1)), EINVAL, "block range [1, 1) of 2"),
    "range past the end": (fork(rng=(0, 3)), EINVAL, "block range [0, 3) of 2"),
    "range negative": (fork(rng=(-1, 2)), EINVAL, "block range [-1, 2) of 2"),
    "range without states": (fork(rng=(1, 2), states=None), EINVAL, "starts from states"),
    "range on the two-pass fork": (fork(Dk=64, Dv=64, rng=(1, 2)), EUNSUP, "block ranges need the pipelined kernel"),
    "range, misaligned rows": (fork(qkv0=P2, rng=(1, 2)), EUNSUP, "block ranges need the pipelined kernel"),
    # fork conv (src/dllm_qwen38/blockdiff.py:167-173, gdn.py:217-219)
    "conv null pointer": (conv(raw0=None), EINVAL, "conv fork: null pointer"),
    "conv empty": (conv(Cd=0), EINVAL, "conv fork: bad sizes"),
    "conv L % block": (conv(L=48), EINVAL, "L=48 is not a multiple of block=32"),
    "conv width 5": (conv(width=5), EUNSUP, "kernel width 5 not supported"),
    "conv width 1": (conv(width=1), EUNSUP, "kernel width 1 not supported"),
    "conv dtype pair": (conv(dw=7), EUNSUP, "dtype pair (1, 7) not supported"),
    "conv grid": (conv(L=32 * 65536), EUNSUP, "grid too large"),
    "conv range reversed": (conv(rng=(2, 1)), EINVAL, "block range [2, 1) of 2"),
    # causal conv ([hf]:219-239)
    "conv1d null pointer": (conv1d(x=None), EINVAL, "causal_conv1d: null pointer"),
    "conv1d width 9": (conv1d(width=9), EINVAL, "bad sizes"),
    "conv1d prefix without data": (conv1d(plen=3), EINVAL, "bad prefix"),
    "conv1d negative prefix": (conv1d(plen=-1), EINVAL, "bad prefix"),
    "conv1d dtype pair": (conv1d(dx=7), EUNSUP, "dtype pair (7, 1) not supported"),
    "conv1d grid": (conv1d(B=70000), EUNSUP, "grid too large"),
    # complementary-mask attention (src/dllm_qwen38/blockdiff.py:50-66,178-182)
    "bd null pointer": (bd(q=None), EINVAL, "attention: null pointer"),
    "bd empty": (bd(L=0), EINVAL, "bad sizes"),
    "bd L % block": (bd(L=48), EINVAL, "L=48 is not a multiple of block=32"),
    "bd GQA ratio": (bd(Hq=5, Hkv=2), EINVAL, "Hq=5 is not a multiple of Hkv=2"),
    "bd head dim": (bd(d=320, st_t=320), EUNSUP, "head_dim 320 > 256"),
    "bd dtype": (bd(dtype=7), EUNSUP, "dtype 7 not supported"),
    "bd 32-bit extent": (bd(L=1 << 15, st_t=1 << 16), EUNSUP, "32-bit element offsets"),
    # the gated attention layer's core in one launch ([hf]:672-698)
    "gated null pointer": (gated(q=None), EINVAL, "gated attention: null pointer"),
    "gated null table": (gated(cos=None), EINVAL, "null rotary table"),
    "gated empty": (gated(B=0), EINVAL, "gated attention: bad sizes"),
    "gated L % block": (gated(L=48), EINVAL, "L=48 is not a multiple of block=32"),
    "gated head dim 32": (gated(d=32, st_t=128), EUNSUP, "fused form needs bf16"),
    "gated rotary 32": (gated(rd=32), EUNSUP, "fused form needs bf16"),
    "gated fp32": (gated(dtype=F32), EUNSUP, "fused form needs bf16"),
    "gated weight dtype": (gated(wdt=7), EUNSUP, "q norm weight dtype 7"),
    "gated misaligned q": (gated(q=P2), EUNSUP, "16-byte aligned"),
    "gated misaligned gate": (gated(gate=P2), EUNSUP, "gate rows must be 8-byte aligned"),
    "k-only prologue without k": (rope(q=None, Hq=0, k=None), EINVAL, "qk norm rope: null pointer"),
    "prologue q heads without q": (rope(q=None), EINVAL, "qk norm rope: null pointer"),
    "prologue negative q heads": (rope(Hq=-1), EINVAL, "qk norm rope: bad sizes"),
    # block-causal attention of the cached decoder (src/dllm_qwen38/decode.py:63-66)
    "bc negative offset": (bc(q0=-1), EINVAL, "bad sizes"),
    "bc offset overflow": (bc(q0=0x7fffffff - 8), EINVAL, "q0 + M overflows"),
    "bc key splits 0": (bc(splits=0), EINVAL, "key_splits=0"),
    "bc key splits 65": (bc(splits=65, ws=P), EINVAL, "key_splits=65"),
    "bc splits without workspace": (bc(splits=4), EINVAL, "need a workspace"),
    "bc GQA ratio": (bc(Hq=3, Hkv=2), EINVAL, "Hq=3 is not a multiple of Hkv=2"),
    # decoder norms, gates and the MLP product ([hf]:168-184,704-737; gdn.py:225-226)
    "rmsnorm null": (("dllm_rmsnorm_fwd", None, None, None, P, P, 4, 64, 1e-6, BF, BF, 1, None), EINVAL,
                     "rmsnorm: null pointer"),
    "rmsnorm dim 0": (("dllm_rmsnorm_fwd", P, None, None, P, P, 4, 0, 1e-6, BF, BF, 1, None), EINVAL, "bad sizes"),
    "rmsnorm sum without residual": (("dllm_rmsnorm_fwd", P, None, P, P, P, 4, 64, 1e-6, BF, BF, 1, None), EINVAL,
                                     "sum_out needs a residual"),
    "rmsnorm dtype pair": (("dllm_rmsnorm_fwd", P, None, None, P, P, 4, 64, 1e-6, F32, BF, 1, None), EUNSUP,
                           "dtype pair (0, 1) not supported"),
    "gated rmsnorm null": (("dllm_gated_rmsnorm_fwd", P, None, P, P, 4, 64, 1e-6, BF, BF, None), EINVAL,
                           "gated rmsnorm: null pointer"),
    "gated rmsnorm dtype pair": (("dllm_gated_rmsnorm_fwd", P, P, P, P, 4, 100, 1e-6, BF, F32, None), EUNSUP,
                                 "dtype pair (1, 0) not supported"),
    "gates null": (("dllm_gdn_gates_fwd", P, P, None, P, P, P, 4, 8, BF, F32, None), EINVAL, "gdn gates: null pointer"),
    "gates no rows": (("dllm_gdn_gates_fwd", P, P, P, P, P, P, 0, 8, BF, F32, None), EINVAL, "bad sizes"),
    "gates dtype pair": (("dllm_gdn_gates_fwd", P, P, P, P, P, P, 4, 8, BF, 7, None), EUNSUP,
                         "dtype pair (1, 7) not supported"),
    "swiglu negative": (("dllm_swiglu_fwd", P, P, P, -1, BF, None), EINVAL, "bad size"),
    "swiglu misaligned": (("dllm_swiglu_fwd", P2, P, P, 64, BF, None), EINVAL, "16-byte aligned"),
    "swiglu dtype": (("dllm_swiglu_fwd", P, P, P, 64, 7, None), EUNSUP, "dtype 7 not supported"),
    # attention prologue ([hf]:554-589,672-680)
    "rope null": (rope(q=None), EINVAL, "qk norm rope: null pointer"),
    "rope odd rotary dim": (rope(rd=15), EINVAL, "bad sizes"),
    "rope rotary past head": (rope(rd=128), EINVAL, "bad sizes"),
    "rope head dim": (rope(hd=512, rd=16), EINVAL, "bad sizes"),
    "rope tables missing": (rope(cos=None), EINVAL, "null rotary table"),
    "rope 32-bit strides": (rope(qst=(1 << 40, 1 << 32, 64)), EUNSUP, "strides exceed 32 bits"),
    "rope dtype pair": (rope(dt=F32, dtw=BF), EUNSUP, "dtype pair (0, 1) not supported"),
    # decoding-step projections
    "linear no projections": (multi(count=0), EINVAL, "0 projections"),
    "linear five projections": (multi(count=5, Ns=(128,) * 5), EINVAL, "5 projections"),
    "linear fp32": (multi(dtype=F32), EUNSUP, "bf16 only"),
    "linear K % 64": (multi(K=96), EUNSUP, "K=96 is not a multiple of 64"),
    "linear misaligned x": (multi(x=P2), EINVAL, "x must be 16-byte aligned"),
    "linear swiglu of one": (multi(swiglu=1), EINVAL, "swiglu takes gate | up of equal N"),
    "linear swiglu unequal": (multi(count=2, Ns=(128, 256), swiglu=1), EINVAL, "swiglu takes gate | up of equal N"),
    "linear empty projection": (multi(count=2, Ns=(128, 0)), EINVAL, "projection 1 is empty"),
    "linear misaligned weights": (multi(w=(P2,)), EINVAL, "weights must be 16-byte aligned"),
    "linear misaligned workspace": (multi(ws=P2), EINVAL, "workspace must be a 16-byte aligned"),
    "linear too many workgroups": (multi(M=64, K=64 * 1024, Ns=(128 * 1024,), wgs=40000), EINVAL,
                                   "40000 workgroups (at most 32768)"),
    "linear rmsnorm no residual": (linrms(r=None), EINVAL, "decode linear rmsnorm: null pointer"),
    "linear rmsnorm no output": (linrms(y=None), EINVAL, "decode linear rmsnorm: null pointer"),
    "linear rmsnorm fp16 weight": (linrms(dtype_w=2), EUNSUP, "norm weight dtype 2"),
    "linear rmsnorm N % 512": (linrms(N=640), EUNSUP, "N=640 is not a multiple of 512"),
    "linear rmsnorm N past 8192": (linrms(N=8704), EUNSUP, "N=8704 is not a multiple of 512 up to 8192"),
    "linear rmsnorm misaligned sum": (linrms(so=P2), EINVAL, "must be 16-byte aligned"),
    "linear rmsnorm 65 rows": (linrms(M=65), EUNSUP, "M=65 > 64 rows"),
    "linear rmsnorm fp32": (linrms(dtype=F32), EUNSUP, "bf16 only"),
    "linear rmsnorm K % 64": (linrms(K=96), EUNSUP, "K=96 is not a multiple of 64"),
    "linear rmsnorm misaligned workspace": (linrms(ws=P2), EINVAL, "workspace must be a 16-byte aligned"),
    "bc gated null gate": (("dllm_block_causal_attention_gated_fwd", P, s3(8, 8, 8), P, s3(8, 8, 8), P, s3(8, 8, 8),
                            None, None, P, 1, 32, 64, 32, 4, 2, 64, 32, 0.125, BF, None, 1, None), EINVAL,
                           "null gate"),
    "bc gated fp32": (("dllm_block_causal_attention_gated_fwd", P, s3(8, 8, 8), P, s3(8, 8, 8), P, s3(8, 8, 8),
                       P, s3(8, 8, 8), P, 1, 32, 64, 32, 4, 2, 64, 32, 0.125, F32, None, 1, None), EUNSUP,
                      "gated form is bf16 only"),
    "bc gated misaligned gate": (("dllm_block_causal_attention_gated_fwd", P, s3(8, 8, 8), P, s3(8, 8, 8), P,
                                  s3(8, 8, 8), P + 4, s3(8, 8, 8), P, 1, 32, 64, 32, 4, 2, 64, 32, 0.125, BF, None, 1,
                                  None), EUNSUP, "gate rows must be 8-byte aligned"),
    "bc gated d 80": (("dllm_block_causal_attention_gated_fwd", P, s3(8, 8, 8), P, s3(8, 8, 8), P, s3(8, 8, 8),
                       P, s3(8, 8, 8), P, 1, 32, 64, 32, 4, 2, 80, 32, 0.125, BF, None, 1, None), EUNSUP,
                      "needs the direct-load kernel"),
    "prologue no mixed output": (prologue(mixed=None), EINVAL, "gdn prologue: null pointer"),
    "prologue T 24": (prologue(T=24), EUNSUP, "T=24 must divide 32"),
    "prologue M not whole sequences": (prologue(M=40, T=16), EUNSUP, "T=16 must divide 32 and M=40"),
    "prologue width 9": (prologue(width=9, plen=8), EUNSUP, "conv width 9"),
    "prologue carry-in length": (prologue(plen=2), EINVAL, "carry-in of 2 positions"),
    "prologue carry-in pointer": (prologue(prefix=None), EINVAL, "carry-in of 3 positions"),
    "prologue b and a differ": (prologue(Ns=(768, 512, 16, 32)), EINVAL, "b and a of 16 and 32 heads"),
    "prologue conv fp16": (prologue(dconv=2), EUNSUP, "conv weight dtype 2"),
    "prologue param fp16": (prologue(dparam=2), EUNSUP, "A_log / dt_bias dtype 2"),
    "prologue projection checks": (prologue(), EUNSUP, "K=96 is not a multiple of 64"),
    "noalloc bad sizes": (("dllm_decode_linear_fwd_noalloc", P, P, P, 0, 128, 128, 4, BF, None), EINVAL, "bad sizes"),
    "noalloc K % 64": (("dllm_decode_linear_fwd_noalloc", P, P, P, 32, 128, 100, 4, BF, None), EUNSUP,
                       "K=100 is not a multiple of 64"),
    # 512 workgroups over 3200 units of 80 k-steps split tiles: 512 x 2 pieces of 16 KB > 8 MiB
    "noalloc past the array": (("dllm_decode_linear_fwd_noalloc", P, P, P, 32, 5120, 5120, 512, BF, None), EUNSUP,
                               "more than the 8388608-byte array"),
    # the fork with the v channels' conv inside, and the conv over the q and k channels only
    "vconv null raw rows": (vfork(raw=None), EINVAL, "gdn fork v conv: null pointer"),
    "vconv weight dtype": (vfork(dtw=7), EUNSUP, "weight dtype 7"),
    "vconv head dim 64": (vfork(Dk=64, Dv=64, stride_t=384), EUNSUP, "needs the pipelined kernel"),
    "vconv fp32": (vfork(dtype=F32), EUNSUP, "needs the pipelined kernel"),
    "vconv misaligned raw rows": (vfork(raw=P2), EUNSUP, "16-byte aligned rows and strides"),
    "vconv misaligned tails": (vfork(tails=P2), EINVAL, "tails need 4-byte alignment"),
    "vconv odd conv_dim": (vfork(cd=767), EINVAL, "tails need 4-byte alignment and an even conv_dim"),
    "vconv block range": (vfork() [:-3] + (1, 1, None), EINVAL, "block range [1, 1)"),
    "conv channels past conv_dim": (convc(128), EINVAL, "y_channels 128 > conv_dim 64"),
    "conv channels negative": (convc(-1), EINVAL, "y_channels -1 < 0"),
    # fork layout (src/dllm_qwen38/blockdiff.py:161-177)
    "layout prefix missing": (("dllm_fork_layout", 1, 64, 32, 4, P, P, None, None), EINVAL, "fork layout: null pointer"),
    "layout width 0": (("dllm_fork_layout", 1, 64, 32, 0, P, P, P, None), EINVAL, "fork layout: bad sizes"),
    "layout rows past 32 bits": (("dllm_fork_layout", 1 << 16, 1 << 20, 16, 4, P, P, P, None), EUNSUP,
                                 "65536 x 65536 fork rows"),
}


@pytest.mark.parametrize("name", list(CASES))
def test_refused_before_launch(name):
    call, code, msg = CASES[name]
    fn = getattr(_lib.lib(), call[0])
    assert fn(*call[1:]) == code, (name, _lib.last_error())
    assert msg in _lib.last_error(), (name, _lib.last_error())


def test_noalloc_limit_is_reported():
    assert _lib.lib().dllm_decode_linear_noalloc_max_bytes() == 8 << 20


def test_empty_inputs_are_accepted_without_a_launch():
    """Zero rows or elements are a valid no-op for the row-wise kernels (what torch does on empty
    tensors); no stream or device is touched."""
    L = _lib.lib()
    assert L.dllm_rmsnorm_fwd(P, None, None, P, P, 0, 64, 1e-6, BF, BF, 1, None) == 0
    assert L.dllm_gated_rmsnorm_fwd(P, P, P, P, 0, 64, 1e-6, BF, BF, None) == 0
    assert L.dllm_swiglu_fwd(P, P, P, 0, BF, None) == 0
    assert L.dllm_swiglu_rows_fwd(P, P, 8, P, 0, 8, BF, None) == 0


@pytest.mark.parametrize("N", range(512, 9216, 512))
def test_fused_norm_widths_agree_with_the_python_gate(N):
    """dllm_decode_linear_rmsnorm_fwd takes exactly the row widths decode._norm_width_fused admits
    (the forward then never sends it a width it refuses): an admitted width gets past the width
    checks and is refused later, on K = 96."""
    from dllm_qwen38_amd import decode

    call = linrms(N=N, K=96)
    rc = getattr(_lib.lib(), call[0])(*call[1:])
    if decode._norm_width_fused(N):
        assert rc == EUNSUP and "K=96 is not a multiple of 64" in _lib.last_error(), (N, _lib.last_error())
    else:
        assert rc == EUNSUP and "decode linear rmsnorm: N=" in _lib.last_error(), (N, _lib.last_error())
