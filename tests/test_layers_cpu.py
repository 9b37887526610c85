"""CPU checks of the host-side layer mirror: weight packing, parameter protocol, option
rejection and device checks (no kernel launches)."""
import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from ae_amd.layers import FusedMoE, MixtralMoE, set_weight_attrs
from ae_amd.layers.topk import check_routing_options


def test_weight_loader_packs_pages_like_the_reference():
    E, H, I = 3, 8, 12
    moe = FusedMoE(num_experts=E, top_k=2, hidden_size=H, intermediate_size=I,
                   params_dtype=torch.float32, tp_size=1)
    assert tuple(moe.ws.shape) == (E, 3 * I * H)
    g = torch.Generator().manual_seed(0)
    mats = {}
    for e in range(E):
        for name, shape in (("w1", (I, H)), ("w2", (H, I)), ("w3", (I, H))):
            mats[e, name] = torch.randn(shape, generator=g)
            moe.weight_loader(moe.ws, mats[e, name], f"model.layers.0.block_sparse_moe.experts.{e}.{name}.weight",
                              name, e)
    for e in range(E):
        want = ref.pack_page(mats[e, "w1"].numpy(), mats[e, "w3"].numpy(), mats[e, "w2"].numpy())
        np.testing.assert_array_equal(moe.ws.data[e].numpy(), want)
        w1, w3, w2 = ref.unpack_page(moe.ws.data[e].numpy(), H, ref.F32)
        np.testing.assert_array_equal(w2, mats[e, "w2"].numpy())


def test_weight_loader_tp_shard(monkeypatch):
    """TP rank r owns rows [r*I_p, (r+1)*I_p) of w1/w3 and those columns of w2."""
    import sys
    fm = sys.modules["ae_amd.layers.FusedMoE"]  # the package attribute is the class
    E, H, I, tp = 1, 4, 8, 2
    monkeypatch.setattr(fm, "_tp_rank_world", lambda: (1, tp))
    moe = FusedMoE(num_experts=E, top_k=1, hidden_size=H, intermediate_size=I,
                   params_dtype=torch.float32, tp_size=tp)
    Ip = I // tp
    w1, w3, w2 = torch.randn(I, H), torch.randn(I, H), torch.randn(H, I)
    for name, wt in (("w1", w1), ("w3", w3), ("w2", w2)):
        moe.weight_loader(moe.ws, wt, f"experts.0.{name}.weight", name, 0)
    want = ref.pack_page(w1[Ip:].numpy(), w3[Ip:].numpy(), w2[:, Ip:].numpy())
    np.testing.assert_array_equal(moe.ws.data[0].numpy(), want)


def test_expert_params_mapping():
    m = FusedMoE.make_expert_params_mapping("w1", "w2", "w3", 2)
    assert m[0] == ("experts.ws", "experts.0.w1.weight", 0, "w1")
    assert m[1] == ("experts.ws", "experts.0.w2.weight", 0, "w2")
    assert m[5] == ("experts.ws", "experts.1.w3.weight", 1, "w3")
    assert len(m) == 6


def test_routing_options():
    from ae_amd.layers.topk import needs_grouped_topk
    with pytest.raises(ValueError):  # sglang asserts both group sizes
        check_routing_options(True, None, 4, None, None, None)
    check_routing_options(True, 2, 4, None, None, None)
    check_routing_options(True, 1, 1, None, None, None)
    check_routing_options(False, None, None, lambda **kw: kw, None, None)  # custom routing
    check_routing_options(True, 2, 4, lambda **kw: kw, torch.zeros(4), None)
    check_routing_options(False, None, None, None, None, 2.5)  # accepted (no effect on top-k)
    with pytest.raises(ValueError):
        check_routing_options(False, None, None, None, None, float("nan"))
    # one group, or all groups selectable, without a bias: the plain top-k of the one-call path
    assert not needs_grouped_topk(False, 2, 4, torch.zeros(4))  # the bias needs the grouped branch
    assert not needs_grouped_topk(True, 1, 1, None)
    assert not needs_grouped_topk(True, 4, 4, None)
    assert needs_grouped_topk(True, 3, 8, None)
    assert needs_grouped_topk(True, 1, 1, torch.zeros(4))
    with pytest.raises(NotImplementedError):
        FusedMoE(4, 2, 8, 8, params_dtype=torch.float32, tp_size=1, quant_config=object())


def test_options_the_reference_ignores_are_accepted():
    """activation, apply_router_weight_on_input, inplace and no_combine are accepted and
    ignored, as the reference's forward_cuda ignores them (specmoe/layers/FusedMoE.py:155-196);
    a non-default value warns once."""
    import warnings
    from ae_amd.layers.FusedMoE import _warned, warn_ignored_options
    moe = FusedMoE(4, 2, 128, 128, params_dtype=torch.bfloat16, tp_size=1, activation="gelu",
                   apply_router_weight_on_input=True, no_combine=True, inplace=False)
    assert moe.no_combine and moe.apply_router_weight_on_input and moe.activation == "gelu"
    _warned.clear()
    with warnings.catch_warnings(record=True) as got:
        warnings.simplefilter("always")
        warn_ignored_options(activation="silu", apply_router_weight_on_input=False, inplace=True,
                             no_combine=False)
        assert not got
        warn_ignored_options(activation="gelu", apply_router_weight_on_input=True, inplace=False,
                             no_combine=True)
        assert len(got) == 4 and all(issubclass(w.category, RuntimeWarning) for w in got)
        warn_ignored_options(activation="gelu", apply_router_weight_on_input=True, inplace=False,
                             no_combine=True)
        assert len(got) == 4  # once per option and value


def test_forward_requires_pool_and_gpu_tensors():
    moe = FusedMoE(4, 2, 128, 128, params_dtype=torch.bfloat16, tp_size=1)
    x = torch.zeros((2, 128), dtype=torch.bfloat16)
    logits = torch.zeros((2, 4), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="pool"):
        moe(x, logits, torch.arange(4))
    set_weight_attrs(moe.ws, {"gpu_cache": torch.zeros((4, 3 * 128 * 128), dtype=torch.bfloat16)})
    with pytest.raises(ValueError, match="GPU"):
        moe(x, logits, torch.arange(4))


def test_mixtral_block_structure():
    blk = MixtralMoE(8, 2, 64, 128, params_dtype=torch.float32, tp_size=1)
    assert blk.gate.weight.shape == (8, 64) and blk.gate.bias is None
    assert blk.experts.renormalize is True and blk.experts.top_k == 2


def test_custom_routing_function_is_called_like_the_reference():
    """select_experts hands a custom routing function the reference's keyword arguments and
    returns its result as fp32 weights / int32 ids (no kernel involved)."""
    from ae_amd.layers import select_experts
    seen = {}

    def route(hidden_states, gating_output, topk, renormalize):
        seen.update(topk=topk, renormalize=renormalize, shape=tuple(gating_output.shape))
        ids = torch.argsort(gating_output, dim=-1, descending=True)[:, :topk]
        return torch.full(ids.shape, 0.5, dtype=torch.float64), ids.to(torch.int64)

    x, logits = torch.randn(5, 8), torch.randn(5, 4)
    w, ids = select_experts(x, logits, 2, renormalize=False, custom_routing_function=route)
    assert seen == {"topk": 2, "renormalize": False, "shape": (5, 4)}
    assert w.dtype == torch.float32 and ids.dtype == torch.int32
    assert torch.equal(ids, torch.argsort(logits, dim=-1, descending=True)[:, :2].to(torch.int32))
