"""GPU parity of the two-stream block-diffusion forward (HIP fork + HIP attention + torch GEMMs).

The oracle is the CPU restatement in oracle/model_ref.py, itself pinned against transformers' own
Qwen3.5 modules. Bars (reference tests/test_equivalence.py uses fork-vs-oracle < 1e-3):
  * fp32 tiny model: fork forward vs the oracle's fork forward and vs the per-block oracle
    <= 1e-4 max-abs on the logits; every fault moves the noised logits by > 1e-3;
  * bf16 tiny model: <= 2^-5 * max|logits| + 2^-6 * |logit| vs the fp32 per-block oracle run on
    the bf16-rounded weights (bf16 activations through 8 layers);
  * 27B-class geometry (hidden 5120, GDN heads 16/48 of dim 128, attention 24/4 of dim 256) at
    full length: the visibility contract as bit-exact invariances (changing a block of x_t moves
    only that block's noised logits; changing a block of x_0 moves nothing before it).
"""

import pytest
import torch

from _tiny import noised_ids, tiny_hf_model
from dllm_qwen38_amd import blockdiff, gdn
from dllm_qwen38_amd import model as hybrid
from oracle import model_ref

pytestmark = pytest.mark.gpu

FAULTS = ("concat-causal-gdn", "mask-leak", "no-conv-prefix")
F32_TOL = 1e-4
FAULT_MIN = 1e-3


@pytest.fixture(scope="module")
def tiny_cpu():
    return tiny_hf_model(seed=0)


@pytest.fixture(scope="module")
def tiny_gpu(tiny_cpu, dev):
    import copy

    model, lm_head = tiny_cpu
    return copy.deepcopy(model).to(dev), copy.deepcopy(lm_head).to(dev)


def _maxdiff(a, b):
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


@pytest.mark.parametrize("B,L,block", [(2, 32, 8), (1, 64, 16), (2, 96, 32), (1, 40, 4)])
def test_fork_forward_fp32_matches_oracles(tiny_cpu, tiny_gpu, dev, B, L, block):
    model, lm_head = tiny_cpu
    gm, gl = tiny_gpu
    x0, xt = noised_ids(B, L, seed=B * 1000 + L + block)
    with torch.no_grad():
        lt, l0 = blockdiff.block_diffusion_forward(gm, gl, x0.to(dev), xt.to(dev), block)
    torch.cuda.synchronize()
    ot, o0 = model_ref.block_diffusion_forward(model, lm_head, x0, xt, block)
    rt = model_ref.reference_block_logits(model, lm_head, x0, xt, block)
    r0 = model_ref.reference_clean_logits(model, lm_head, x0, block)
    d = [_maxdiff(lt, ot), _maxdiff(l0, o0), _maxdiff(lt, rt), _maxdiff(l0, r0)]
    print(f"B{B} L{L} block{block}: fork-vs-oracle t={d[0]:.2e} 0={d[1]:.2e}  per-block t={d[2]:.2e} 0={d[3]:.2e}")
    assert max(d) <= F32_TOL


@pytest.mark.parametrize("fault", FAULTS)
def test_faults_match_oracle_fault_and_break_equivalence(tiny_cpu, tiny_gpu, dev, fault):
    model, lm_head = tiny_cpu
    gm, gl = tiny_gpu
    x0, xt = noised_ids(2, 32, seed=7)
    with torch.no_grad():
        lt, _ = blockdiff.block_diffusion_forward(gm, gl, x0.to(dev), xt.to(dev), 8,
                                                  fault=blockdiff.BreakMode(fault))
    torch.cuda.synchronize()
    ot, _ = model_ref.block_diffusion_forward(model, lm_head, x0, xt, 8, fault=fault)
    rt = model_ref.reference_block_logits(model, lm_head, x0, xt, 8)
    print(f"{fault}: vs oracle-with-fault {_maxdiff(lt, ot):.2e}, vs per-block oracle {_maxdiff(lt, rt):.2e}")
    assert _maxdiff(lt, ot) <= F32_TOL
    assert _maxdiff(lt, rt) > FAULT_MIN


def test_hidden_output_layers_and_layer_step_module(tiny_cpu, tiny_gpu, dev):
    model, lm_head = tiny_cpu
    gm, gl = tiny_gpu
    x0, xt = noised_ids(1, 32, seed=8)
    x0d, xtd = x0.to(dev), xt.to(dev)
    with torch.no_grad():
        ht, h0 = blockdiff.block_diffusion_forward(gm, gl, x0d, xtd, 8, output="hidden", layers=5)
        # the same stack through LayerStep modules (the FSDP unit); pos shaped like HF's rotary
        # output [B, 2L, rotary_dim] for positions (i mod L), which it must also agree with
        a0, at = gm.embed_tokens(x0d), gm.embed_tokens(xtd)
        c1, s1 = blockdiff.rotary_tables(gm, 32, dev, torch.float32)
        cos, sin = torch.cat([c1, c1])[None], torch.cat([s1, s1])[None]
        pos = torch.arange(64, device=dev).view(1, 1, -1).expand(3, 1, -1)
        hc, hs = gm.rotary_emb(a0, pos % 32)
        assert max(_maxdiff(hc, cos), _maxdiff(hs, sin)) <= 1e-6
        for i in range(5):
            a0, at = blockdiff.LayerStep(gm.layers[i], gm.config.layer_types[i])(a0, at, (cos, sin), None, 8)
        at, a0 = blockdiff.rmsnorm(at, gm.norm), blockdiff.rmsnorm(a0, gm.norm)
    torch.cuda.synchronize()
    rt, r0 = model_ref.block_diffusion_forward(model, lm_head, x0, xt, 8, output="hidden", layers=5)
    assert ht.shape == (1, 32, 64)
    assert max(_maxdiff(ht, rt), _maxdiff(h0, r0)) <= F32_TOL
    assert torch.equal(at, ht) and torch.equal(a0, h0)
    with pytest.raises(ValueError):
        blockdiff.LayerStep(gm.layers[0], "linear_attention")(a0, at, (cos, sin), torch.zeros(1), 8)


def test_forward_refuses_autograd(tiny_gpu, dev):
    gm, gl = tiny_gpu
    x0, xt = noised_ids(1, 16, seed=9)
    gl.weight.requires_grad_(True)
    try:
        with pytest.raises(RuntimeError, match="forward-only"):
            blockdiff.block_diffusion_forward(gm, gl, x0.to(dev), xt.to(dev), 8)
    finally:
        gl.weight.requires_grad_(False)


def test_bf16_tiny_model_within_bound(tiny_cpu, tiny_gpu, dev):
    import copy

    model, lm_head = tiny_cpu
    gm, gl = (copy.deepcopy(m).to(dev, torch.bfloat16) for m in tiny_cpu)
    # the fp32 oracle on the same (bf16-rounded) weights
    om, ol = (copy.deepcopy(m).to(torch.bfloat16).float() for m in tiny_cpu)
    x0, xt = noised_ids(2, 64, seed=10)
    with torch.no_grad():
        lt, l0 = blockdiff.block_diffusion_forward(gm, gl, x0.to(dev), xt.to(dev), 16)
    torch.cuda.synchronize()
    rt = model_ref.reference_block_logits(om, ol, x0, xt, 16)
    r0 = model_ref.reference_clean_logits(om, ol, x0, 16)
    for got, ref, name in ((lt, rt, "t"), (l0, r0, "0")):
        err = (got.float().cpu() - ref).abs()
        bound = 2 ** -5 * ref.abs().max().item() + 2 ** -6 * ref.abs()
        print(f"bf16 stream {name}: max|d|={err.max().item():.3e} max|ref|={ref.abs().max().item():.3e}")
        assert (err <= bound).all(), name


@pytest.fixture(scope="module")
def stack27(dev):
    """4 layers (3 GDN + 1 attention) of the 27B-class geometry, bf16, vocab cut to 4096 (the
    embedding and lm_head are not on the path), seeded N(0, 0.02) init on the device."""
    c = hybrid.config_27b_truncated(layers=4)
    c.vocab_size = 4096
    model, lm_head = hybrid.build(c, device=dev, dtype=torch.bfloat16, seed=13)
    model.requires_grad_(False)
    lm_head.requires_grad_(False)
    return model, lm_head


def test_27b_class_visibility_invariances_bit_exact(stack27, dev):
    model, lm_head = stack27
    B, L, block = 1, 2048, 32
    x0, xt = noised_ids(B, L, vocab=4096, seed=11)
    x0, xt = x0.to(dev), xt.to(dev)
    k = 17
    sl = slice(k * block, (k + 1) * block)
    xt2 = xt.clone()
    xt2[:, sl] = (xt2[:, sl] + 1) % 4096
    x02 = x0.clone()
    x02[:, sl] = (x02[:, sl] + 7) % 4096
    with torch.no_grad():
        lt, l0 = blockdiff.block_diffusion_forward(model, lm_head, x0, xt, block)
        lt_b, l0_b = blockdiff.block_diffusion_forward(model, lm_head, x0, xt2, block)
        lt_c, l0_c = blockdiff.block_diffusion_forward(model, lm_head, x02, xt, block)
        lt_r, l0_r = blockdiff.block_diffusion_forward(model, lm_head, x0, xt, block)
    torch.cuda.synchronize()
    assert torch.isfinite(lt).all() and torch.isfinite(l0).all()
    assert torch.equal(lt, lt_r) and torch.equal(l0, l0_r), "run-to-run determinism"
    # x_t block k changed: the clean stream and every other noised block are bit-identical
    assert torch.equal(l0_b, l0)
    assert torch.equal(lt_b[:, : k * block], lt[:, : k * block])
    assert torch.equal(lt_b[:, (k + 1) * block:], lt[:, (k + 1) * block:])
    assert not torch.equal(lt_b[:, sl], lt[:, sl])
    # x_0 block k changed: nothing before it moves; noised blocks <= k see only x_0 blocks < k
    assert torch.equal(l0_c[:, : k * block], l0[:, : k * block])
    assert torch.equal(lt_c[:, : (k + 1) * block], lt[:, : (k + 1) * block])
    assert not torch.equal(lt_c[:, (k + 1) * block:], lt[:, (k + 1) * block:])


def test_equivalence_harness_passes_and_detects_every_fault(dev, tmp_path):
    """The reference's harness contract on the HIP path: 5/5 checks, 3/3 faults, exit 0."""
    import json

    from dllm_qwen38_amd import equivalence

    out = tmp_path / "eq.json"
    assert equivalence.main(["--block", "8", "--nblocks", "4", "--json", str(out)]) == 0
    rep = json.loads(out.read_text())
    assert rep["checks_passed"] == rep["checks_total"] == 5
    assert rep["faults_detected"] == rep["faults_total"] == 3
    out16 = tmp_path / "eq16.json"
    assert equivalence.main(["--dtype", "bfloat16", "--block", "16", "--nblocks", "4", "--change-floor", "1e-3",
                             "--json", str(out16)]) == 0


def test_batched_forward_equals_per_row_and_oracle(dev):
    """The reference's structural check (tests/test_equivalence.py:30-47) on the HIP path: B = 3
    rows in one forward equal three one-row forwards, and match the per-block oracle."""
    model, lm_head = tiny_hf_model(seed=2)
    import copy

    gm, gl = copy.deepcopy(model).to(dev), copy.deepcopy(lm_head).to(dev)
    block, nb, B = 8, 3, 3
    g = torch.Generator().manual_seed(2)
    x0 = torch.randint(0, 256, (B, block * nb), generator=g)
    xt = x0.clone()
    xt[torch.rand(B, block * nb, generator=g) < 0.5] = 255
    with torch.no_grad():
        lt, l0 = blockdiff.block_diffusion_forward(gm, gl, x0.to(dev), xt.to(dev), block)
        rows = [blockdiff.block_diffusion_forward(gm, gl, x0[i:i + 1].to(dev), xt[i:i + 1].to(dev), block)[0]
                for i in range(B)]
    torch.cuda.synchronize()
    ref = model_ref.reference_block_logits(model, lm_head, x0, xt, block)
    assert lt.shape == (B, block * nb, 256)
    d_rows, d_ref = _maxdiff(lt, torch.cat(rows, 0)), _maxdiff(lt, ref)
    print(f"batched vs per-row {d_rows:.2e}, vs per-block oracle {d_ref:.2e}")
    assert d_rows < 1e-5
    assert d_ref < F32_TOL


def test_gdn_mixer_need_states_false_matches_true(tiny_gpu, dev):
    """gdn_mixer_forward with need_states True/False (reference tests/test_equivalence.py:68-84):
    bitwise-equal outputs, states [B, n_chunks, Hv, Dk, Dv] or None, raw_qkv of equal shape."""
    gm, _ = tiny_gpu
    m = gm.layers[0].linear_attn
    hs = torch.randn(2, 16, gm.config.hidden_size, generator=torch.Generator().manual_seed(4)).to(dev)
    with torch.no_grad():
        o1, s1, raw1 = gdn.gdn_mixer_forward(m, hs, chunk_size=16, need_states=True)
        o2, s2, raw2 = gdn.gdn_mixer_forward(m, hs, chunk_size=16, need_states=False)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert s1.shape == (2, 1, m.num_v_heads, m.head_k_dim, m.head_v_dim)
    assert s2 is None
    assert raw1.shape == raw2.shape == (2, m.conv_dim, 16)
    assert gdn.last_impl()[0] == "hip"


@pytest.mark.parametrize("chunk", [8, 16])
def test_gdn_mixer_prefix_and_initial_state_vs_oracle(tiny_cpu, tiny_gpu, dev, chunk):
    """gdn_mixer_forward with a conv prefix and an initial state, as the fork's noised rows call it
    (reference blockdiff.py:174-176), against the oracle mixer on the CPU."""
    model, _ = tiny_cpu
    gm, _ = tiny_gpu
    m_cpu, m = model.layers[1].linear_attn, gm.layers[1].linear_attn
    g = torch.Generator().manual_seed(40 + chunk)
    B, T = 3, 32
    hs = torch.randn(B, T, gm.config.hidden_size, generator=g)
    pre = torch.randn(B, m.conv_dim, m.conv_kernel_size - 1, generator=g)
    init = 0.5 * torch.randn(B, m.num_v_heads, m.head_k_dim, m.head_v_dim, generator=g)
    with torch.no_grad():
        o, st, raw = gdn.gdn_mixer_forward(m, hs.to(dev), chunk_size=chunk, conv_prefix=pre.to(dev),
                                           initial_state=init.to(dev))
        ro, rst, rraw = model_ref.gdn_mixer(m_cpu, hs, chunk=chunk, conv_prefix=pre, initial_state=init)
    torch.cuda.synchronize()
    d = (_maxdiff(o, ro), _maxdiff(st, rst), _maxdiff(raw, rraw))
    print(f"chunk {chunk}: out {d[0]:.2e} states {d[1]:.2e} raw {d[2]:.2e}")
    assert max(d) <= F32_TOL
    # the prefix and the initial state both matter here
    with torch.no_grad():
        o_cold, _, _ = gdn.gdn_mixer_forward(m, hs.to(dev), chunk_size=chunk)
    assert _maxdiff(o, o_cold) > FAULT_MIN


def test_equivalence_harness_layer_truncation_and_report(dev, tmp_path):
    """--layers N runs the first N layers only and says so (reference tests/test_equivalence.py:
    22-27); the report names the oracle's attention backend and GDN core."""
    import json

    from dllm_qwen38_amd import equivalence

    out = tmp_path / "eq3.json"
    rc = equivalence.main(["--layers", "3", "--block", "8", "--nblocks", "2", "--seed", "1", "--change-floor", "0.05",
                           "--attn", "sdpa", "--json", str(out)])
    rep = json.loads(out.read_text())
    assert rep["layers"] == 3
    assert rep["layer_types"] == ["linear_attention"] * 3
    assert rep["checks_passed"] == rep["checks_total"] == 5
    # three GDN layers hold no attention layer, so the mask-leak fault has nothing to break and the
    # harness reports it undetected (exit 1) rather than claiming a detection it cannot make
    assert [f["fault"] for f in rep["faults"] if not f["detected"]] == ["mask-leak"]
    assert rc == 1
    assert rep["attn"] == "sdpa"
    assert rep["oracle_gdn_kernel"] == "torch-reference"
