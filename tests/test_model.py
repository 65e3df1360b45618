"""Host logic of the GraniteMoE-shaped model (CPU, torch reference MoE):
KV-cache decoding equals full recomputation, teacher forcing reproduces
greedy decoding, configs load by the reference's field names."""
import json

import pytest
import torch

from miniep_amd.model import (GraniteMoeModel, KVCache, ModelConfig, greedy_generate, layer_keys,
                              random_weights)
from torch_moe_ref import TorchMoERef, torch_route

TINY = ModelConfig(hidden_size=64, intermediate_size=32, num_hidden_layers=2, num_attention_heads=4,
                   num_key_value_heads=2, num_local_experts=4, num_experts_per_tok=2, vocab_size=97,
                   max_position_embeddings=64)


def _tiny_model(seed=0):
    w = random_weights(TINY, seed=seed, dtype=torch.float32, std=0.2)
    moe = [TorchMoERef(w[layer_keys(i)["w_in"]], w[layer_keys(i)["w_out"]]) for i in range(TINY.num_hidden_layers)]
    return GraniteMoeModel(TINY, w, torch_route, moe)


def test_incremental_decode_equals_full_forward():
    m = _tiny_model()
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(1, TINY.vocab_size, (3, 20), generator=g)
    full = m(ids)                                            # (3, 20, V), causal, no cache
    cache = KVCache(TINY, 3, 20, "cpu")
    parts = [m(ids[:, :12], cache=cache)]
    for t in range(12, 20):
        parts.append(m(ids[:, t:t + 1], cache=cache))
    inc = torch.cat(parts, dim=1)
    assert cache.length == 20
    torch.testing.assert_close(inc, full, rtol=1e-4, atol=1e-4)


def test_logits_at_and_teacher_forcing():
    m = _tiny_model(1)
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(1, TINY.vocab_size, (2, 9), generator=g)
    last = m(ids, logits_at=torch.tensor([8, 8]))
    torch.testing.assert_close(last[:, 0], m(ids)[:, 8], rtol=1e-5, atol=1e-5)
    toks, margins = greedy_generate(m, ids, 6)
    assert toks.shape == (2, 6) and (margins >= 0).all()
    again, _ = greedy_generate(m, ids, 6, forced=toks)
    assert torch.equal(again, toks)
    # greedy tokens are the argmax of a full recomputation at every step
    seq = torch.cat([ids, toks[:, :-1]], dim=1)
    ref = m(seq)[:, 8:].argmax(-1)
    assert torch.equal(ref, toks)


def test_kv_cache_overflow_and_backend_count():
    cache = KVCache(TINY, 1, 4, "cpu")
    m = _tiny_model()
    m(torch.ones(1, 4, dtype=torch.long), cache=cache)
    with pytest.raises(ValueError, match="KV cache full"):
        m(torch.ones(1, 1, dtype=torch.long), cache=cache)
    with pytest.raises(ValueError, match="MoE backends"):
        GraniteMoeModel(TINY, m.w, torch_route, m.moe[:1])


def test_config_from_reference_field_names(tmp_path):
    raw = {f: getattr(TINY, f) for f in TINY.__dataclass_fields__}
    raw["model_type"] = "granitemoe"                        # extra checkpoint keys are ignored
    p = tmp_path / "config.json"
    p.write_text(json.dumps(raw))
    cfg = ModelConfig.from_json(p)
    assert cfg == TINY and cfg.head_dim == 16


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_torch_moe_ref_pinned_against_oracle(dtype):
    """TorchMoERef and torch_route, the reference MoE block of the full-model
    tests, against the numpy oracle (router_logits + topk_softmax,
    moe_layer_local) on tie-free rows with masked tokens, fp32 (bar 1e-5) and
    bf16 (act and expert outputs rounded to bf16; bar 2e-2 normwise and per
    row).  A planted mutant -- gate and up halves swapped -- must fail the bar."""
    import numpy as np

    from helpers import TOL_BF16, TOL_F32, rel_err, row_rel_err, tie_free
    from oracle import moe_oracle as O

    g = torch.Generator().manual_seed(7)
    n, H, inter, E, k = 96, 128, 64, 8, 2
    x = torch.randn(n, H, generator=g).to(dtype)
    w_r = (torch.randn(E, H, generator=g) * 0.1).to(dtype)
    w_in = (torch.randn(E, 2 * inter, H, generator=g) * 0.05).to(dtype)
    w_out = (torch.randn(E, H, inter, generator=g) * 0.05).to(dtype)
    valid = torch.rand(n, generator=g) < 0.8
    bf = dtype == torch.bfloat16
    xf, wrf, wif, wof = (t.float().numpy() for t in (x, w_r, w_in, w_out))

    idx, gate = torch_route(x, w_r, k)
    lg = O.router_logits(xf, wrf)
    assert tie_free(lg, k)
    oidx, ogate = O.topk_softmax(lg, k, gate_bf16=bf)
    assert np.array_equal(idx.numpy(), oidx)
    np.testing.assert_allclose(gate.float().numpy(), ogate, rtol=1e-2 if bf else 1e-6, atol=0)

    want = O.moe_layer_local(xf, oidx, gate.float().numpy(), wif, wof, valid.numpy(), act_bf16=bf, out_bf16=bf)
    got = TorchMoERef(w_in, w_out)(x, idx, gate, valid).float().numpy()
    tol = TOL_BF16 if bf else TOL_F32
    assert (got[~valid.numpy()] == 0).all()
    assert rel_err(got, want) <= tol
    assert row_rel_err(got[valid.numpy()], want[valid.numpy()], floor=1e-3 * float(np.abs(want).max())) <= tol
    swapped = torch.cat([w_in[:, inter:], w_in[:, :inter]], dim=1)
    bad = TorchMoERef(swapped, w_out)(x, idx, gate, valid).float().numpy()
    assert rel_err(bad, want) > 10 * tol
