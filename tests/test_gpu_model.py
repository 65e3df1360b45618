"""Config 3: 24-layer GraniteMoE-shaped model (hidden 1024, 16 q / 8 kv heads
of 64, RoPE, RMSNorm, vocab 49155, 32 experts top-8 per layer), seeded
random-init weights, prefill 8 x 512 seeded random token ids, then 32 greedy
steps with every MoE block on the HIP kernels, against the same model with
the torch restatement of the reference router + LocalMoEBackend
(modeling.py:131-145,186-197) in every layer.  Greedy identity is the
reference's own gate (worker.py:165-173, modeling.py:249-262).

Expert weights are drawn larger than the other matrices so that every MoE
block moves the residual stream by O(1): N(0, 0.06) / N(0, 0.12)
(input_linear / output_linear) in fp32, N(0, 0.05) / N(0, 0.1) in bf16.  With
N(0, 0.02) everywhere -- and in fp32 still with (0.05, 0.1) -- the random model
mostly repeats its input token, its greedy choices hardly depend on the MoE
blocks, and identity would hold trivially.  Each test shows that they do
depend on them here: scaling one layer's MoE output by 0.9 moves a fifth of
the decoded tokens or more.  (In bf16 at the fp32 scale the model is so
chaotic that one-ulp rounding differences decide about 40 % of the
teacher-forced decisions: its logits are about 0.5 in size, top-2 gaps about
0.02, and the step's logit error about 0.1.)

fp32: the HIP fp32 kernels against the fp32 restatement; the 8 x 32
continuations must be identical.

bf16: the two paths legitimately round differently (one bf16 ulp in some
expert outputs: their fp32 sums run in different orders), and a random
24-layer model whose MoE blocks matter amplifies that.  Both models are
teacher-forced on the HIP model's tokens, so every step sees the same prefix;
a decision may then differ only where the reference's top-2 logit gap is
below the logit error measured at that very step (every such decision is
printed); the free-running continuations are reported.
"""
import time

import pytest
import torch

from helpers import banner
from miniep_amd.model import GraniteMoeModel, ModelConfig, build_hip_model, greedy_generate, layer_keys, random_weights
from torch_moe_ref import TorchMoERef, torch_route

pytestmark = pytest.mark.gpu
DEV = "cuda"
EXPERT_STD = {torch.float32: (0.06, 0.12), torch.bfloat16: (0.05, 0.1)}


class _Scaled:
    """A MoE backend whose output is scaled (the sensitivity probe)."""

    def __init__(self, inner, factor):
        self.inner, self.factor = inner, factor

    def __call__(self, *a, **kw):
        return self.inner(*a, **kw) * self.factor


def _ref_model(cfg, w):
    return GraniteMoeModel(cfg, w, torch_route,
                           [TorchMoERef(w[layer_keys(i)["w_in"]], w[layer_keys(i)["w_out"]])
                            for i in range(cfg.num_hidden_layers)])


def _setup(dtype, seed=0):
    cfg = ModelConfig()
    w = random_weights(cfg, seed=seed, dtype=dtype, device=DEV, expert_std=EXPERT_STD[dtype])
    hip = build_hip_model(cfg, w, check=True)
    ref = _ref_model(cfg, w)
    g = torch.Generator().manual_seed(1)
    prompts = torch.randint(1, cfg.vocab_size, (8, 512), generator=g).to(DEV)
    return cfg, w, hip, ref, prompts


def _sensitivity(ref, prompts, ref_free):
    """Decisions moved when layer 12's MoE output is scaled by 0.9."""
    ref.moe[12] = _Scaled(ref.moe[12], 0.9)
    ptoks, _ = greedy_generate(ref, prompts, 32)
    ref.moe[12] = ref.moe[12].inner
    return int((ptoks != ref_free).sum())


def test_config3_fp32_greedy_identity():
    banner("config 3 fp32: 24 layers, prefill 8x512, 32 greedy steps, identity")
    cfg, w, hip, ref, prompts = _setup(torch.float32)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks, _, hip_logits = greedy_generate(hip, prompts, 32, return_logits=True)
    torch.cuda.synchronize()
    t_hip = time.perf_counter() - t0
    rtoks, rmargins = greedy_generate(ref, prompts, 32)
    # the same steps teacher-forced on the HIP tokens: the logit error of the fp32 path
    _, _, ref_logits = greedy_generate(ref, prompts, 32, forced=toks, return_logits=True)
    err = (hip_logits - ref_logits).abs().amax(-1)
    moved = _sensitivity(ref, prompts, rtoks)
    same_rows = int((toks == rtoks).all(1).sum())
    print(f"fp32 HIP model: prefill + 32 steps in {t_hip:.2f} s; identical sequences {same_rows}/8; "
          f"teacher-forced logit error max {float(err.max()):.3e} (median {float(err.median()):.3e}); "
          f"smallest reference top-2 gap {float(rmargins.min()):.3e}; layer-12 MoE x0.9 moves "
          f"{moved}/{toks.numel()}", flush=True)
    assert moved > toks.numel() // 5, "the decoded tokens do not depend on the MoE blocks"
    assert torch.equal(toks, rtoks), "fp32 greedy continuations differ from the reference"


def test_config3_bf16_greedy():
    banner("config 3 bf16: 24 layers, prefill 8x512, 32 greedy steps")
    cfg, w, hip, ref, prompts = _setup(torch.bfloat16)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks, _, hip_logits = greedy_generate(hip, prompts, 32, return_logits=True)
    torch.cuda.synchronize()
    t_hip = time.perf_counter() - t0
    # the reference teacher-forced on the HIP model's tokens: same prefix at every step
    rtoks, rmargins, ref_logits = greedy_generate(ref, prompts, 32, forced=toks, return_logits=True)
    err = (hip_logits - ref_logits).abs().amax(-1)                       # (8, 32) logit error per step
    scale = ref_logits.abs().amax(-1)
    rel = err / scale
    differ = toks != rtoks
    ref_free, _ = greedy_generate(ref, prompts, 32)
    moved = _sensitivity(ref, prompts, ref_free)
    for b, s in differ.nonzero().tolist():
        print(f"  decision (seq {b}, step {s}): HIP {int(toks[b, s])} vs reference {int(rtoks[b, s])}, "
              f"reference top-2 gap {float(rmargins[b, s]):.4f}, logit error at that step {float(err[b, s]):.4f}",
              flush=True)
    print(f"bf16 HIP model: prefill + 32 steps in {t_hip:.2f} s; teacher-forced decisions differing "
          f"{int(differ.sum())}/{toks.numel()}; logit error per step: median {float(err.median()):.4f} "
          f"(rel {float(rel.median()):.2e}), max {float(err.max()):.4f} (rel {float(rel.max()):.2e}); "
          f"free-running sequences identical {int((toks == ref_free).all(1).sum())}/8; layer-12 MoE x0.9 "
          f"moves {moved}/{toks.numel()}", flush=True)
    assert moved > toks.numel() // 5, "the decoded tokens do not depend on the MoE blocks"
    assert bool((rmargins[differ] < err[differ]).all()), \
        "a decision differs where the reference's top-2 gap exceeds the logit error at that step"
    assert int(toks.min()) >= 0 and int(toks.max()) < cfg.vocab_size


def test_config3_prefill_logits_close():
    banner("config 3: prefill logits vs torch reference (4 layers)")
    cfg = ModelConfig(num_hidden_layers=4)
    w = random_weights(cfg, seed=2, dtype=torch.bfloat16, device=DEV, expert_std=EXPERT_STD[torch.bfloat16])
    hip = build_hip_model(cfg, w)
    ref = _ref_model(cfg, w)
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(1, cfg.vocab_size, (2, 256), generator=g).to(DEV)
    at = torch.full((2,), 255, device=DEV)
    a, b = hip(ids, logits_at=at), ref(ids, logits_at=at)
    err = float((a - b).abs().max() / b.abs().max())
    print(f"last-position logits rel err {err:.3e}", flush=True)
    assert err < 2e-2
    assert torch.equal(a.argmax(-1), b.argmax(-1))
