"""Architecture inference and the routing flags it hands HybridMoE, on the CPU.

Restates the reference's own config tests with fake HF configs
(nano_ktrans tests/test_core.py:236-270 for Qwen2-MoE, :298-329 for Qwen3-MoE)
for the fields on the expert path, plus the ``norm_topk_prob`` override of
nano_ktrans/models/config.py:126, 181: Qwen3-30B-A3B's HF config says
``norm_topk_prob: true``, which overrides the Qwen3 spec's default (False),
and a wrong override silently flips renormalisation on that layer.  The last
test routes one row of logits with each architecture's flags through the
oracle, so a flag mapped to the wrong meaning shows as wrong weights."""
from types import SimpleNamespace

import numpy as np
import pytest

import oracle as O
from nano_ktrans_amd.models.config import (MIXTRAL_SPEC, QWEN2_MOE_SPEC, QWEN3_MOE_SPEC, infer_architecture,
                                           routing_flags)


def _qwen2_moe(**over):
    # the fields of test_core.py:238-260 that reach the expert path
    cfg = dict(model_type="qwen2_moe", architectures=["Qwen2MoeForCausalLM"], hidden_size=2048,
               intermediate_size=5632, moe_intermediate_size=1408, shared_expert_intermediate_size=5632,
               num_experts=60, num_experts_per_tok=4, hidden_act="silu")
    cfg.update(over)
    return SimpleNamespace(**cfg)


def _qwen3_moe(**over):
    # test_core.py:300-318, plus norm_topk_prob where a case sets it
    cfg = dict(model_type="qwen3_moe", architectures=["Qwen3MoeForCausalLM"], hidden_size=2048,
               intermediate_size=6144, moe_intermediate_size=768, num_experts=128, num_experts_per_tok=8,
               hidden_act="silu")
    cfg.update(over)
    return SimpleNamespace(**cfg)


def _mixtral(**over):
    cfg = dict(model_type="mixtral", architectures=["MixtralForCausalLM"], hidden_size=4096,
               intermediate_size=14336, num_local_experts=8, num_experts_per_tok=2, hidden_act="silu")
    cfg.update(over)
    return SimpleNamespace(**cfg)


def test_qwen2_moe_mapping():
    hf = _qwen2_moe()
    assert infer_architecture(hf) is QWEN2_MOE_SPEC
    f = routing_flags(hf)
    assert f["router_use_softmax"] is True
    assert f["normalize_topk_prob"] is False  # Qwen1.5-MoE: no top-k renormalisation
    assert f["experts_are_packed"] is False
    assert f["expert_key_template"] == "model.layers.{layer}.mlp.experts.{expert}.{proj}_proj.weight"
    assert f["expert_proj_names"] == {"gate": "gate", "up": "up", "down": "down"}
    assert QWEN2_MOE_SPEC.has_shared_expert
    assert QWEN2_MOE_SPEC.shared_expert_gate_prefix == "mlp.shared_expert_gate"


def test_qwen3_moe_mapping_and_norm_topk_prob_override():
    # without the HF field: the spec default (no renormalisation)
    plain = _qwen3_moe()
    assert infer_architecture(plain) is QWEN3_MOE_SPEC
    assert QWEN3_MOE_SPEC.use_qk_norm and QWEN3_MOE_SPEC.experts_are_packed
    f = routing_flags(plain)
    assert f["router_use_softmax"] is True
    assert f["normalize_topk_prob"] is False
    assert f["experts_are_packed"] is True
    assert f["expert_proj_names"] == {"gate_up": "gate_up_proj", "down": "down_proj"}
    # Qwen3-30B-A3B's config.json: norm_topk_prob = true overrides the spec
    assert routing_flags(_qwen3_moe(norm_topk_prob=True))["normalize_topk_prob"] is True
    # an explicit false stays false; None means "not set"
    assert routing_flags(_qwen3_moe(norm_topk_prob=False))["normalize_topk_prob"] is False
    assert routing_flags(_qwen3_moe(norm_topk_prob=None))["normalize_topk_prob"] is False
    # the override is per config, never written back into the shared spec
    assert QWEN3_MOE_SPEC.normalize_topk_prob is False


def test_override_applies_to_every_architecture():
    assert routing_flags(_qwen2_moe(norm_topk_prob=True))["normalize_topk_prob"] is True
    assert routing_flags(_mixtral(norm_topk_prob=False))["normalize_topk_prob"] is False
    assert routing_flags(_mixtral())["normalize_topk_prob"] is True


def test_mixtral_mapping():
    hf = _mixtral()
    assert infer_architecture(hf) is MIXTRAL_SPEC
    f = routing_flags(hf)
    assert f["router_use_softmax"] is False  # top-k on the logits, then softmax over the k
    assert f["normalize_topk_prob"] is True
    assert f["expert_proj_names"] == {"gate": "w1", "up": "w3", "down": "w2"}


@pytest.mark.parametrize("hf,spec", [
    # matched by the architectures list when model_type is missing or foreign
    (SimpleNamespace(model_type="", architectures=["Qwen2MoeForCausalLM"]), QWEN2_MOE_SPEC),
    (SimpleNamespace(model_type="custom", architectures=["Qwen3MoeForCausalLM"]), QWEN3_MOE_SPEC),
    # an unknown model with a shared expert is read as Qwen2-MoE, anything else as Mixtral
    (SimpleNamespace(model_type="custom", architectures=[], shared_expert_intermediate_size=4096), QWEN2_MOE_SPEC),
    (SimpleNamespace(model_type="deepseek_v2", architectures=["DeepseekV2ForCausalLM"]), MIXTRAL_SPEC),
    (SimpleNamespace(model_type="custom", architectures=None), MIXTRAL_SPEC),
])
def test_inference_fallbacks(hf, spec):
    """config.py:204-220: model_type first, then the architectures list, then
    the shared-expert field, then Mixtral."""
    assert infer_architecture(hf) is spec


def test_flags_route_as_their_architecture():
    """One row of logits routed with each architecture's flags (the oracle's
    K1): Qwen3-30B-A3B (softmax, renormalised) gives k weights summing to one;
    Qwen1.5-MoE (softmax, not renormalised) gives the raw top-k softmax
    probabilities, summing to less than one; Mixtral (top-k of the logits,
    then softmax over the k) gives the same ids as the softmax arches and
    weights equal to the renormalised probabilities up to fp32 rounding."""
    rng = np.random.default_rng(3)
    logits = rng.standard_normal((1, 16)).astype(np.float32)
    k = 4

    def route(hf):
        f = routing_flags(hf)
        return O.route(logits, k, f["router_use_softmax"], f["normalize_topk_prob"], False)

    ids3, w3 = route(_qwen3_moe(norm_topk_prob=True))
    ids2, w2 = route(_qwen2_moe())
    idsm, wm = route(_mixtral())
    want = np.argsort(-logits[0], kind="stable")[:k]
    for ids in (ids3, ids2, idsm):
        assert sorted(ids[0].tolist()) == sorted(want.tolist())
    assert abs(float(w3.sum()) - 1.0) < 1e-6
    p = np.exp(logits[0].astype(np.float64) - logits[0].max())
    p /= p.sum()
    np.testing.assert_allclose(np.sort(w2[0]), np.sort(p[want]), rtol=1e-6)
    assert float(w2.sum()) < 1.0 - 1e-3
    np.testing.assert_allclose(np.sort(wm[0]), np.sort(p[want] / p[want].sum()), rtol=1e-5)
