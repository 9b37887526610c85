"""The timed CPU baselines (oracle/torch_cpu.py, torch on MKL; oracle/cpu_moe.cpp, cblas_sgemm on
MKL) against the numpy oracle: same routing ids, weights within fp32 rounding, outputs within
the parity tolerance -- so the baselines bench.py times compute the same layer."""
import numpy as np
import pytest
import torch

from oracle import moe_ref as ref
from oracle.torch_cpu import TorchCpuMoE
from tests.golden.synth import make_case
from tests.helpers import TOL_BY_NAME, parity


def _check(case, name):
    x = torch.from_numpy(ref.to_f32(case["x"], case["dtype"]))
    logits = torch.from_numpy(np.asarray(case["logits"], np.float32))
    moe = TorchCpuMoE(case["pool"], case["slot_map"], case["H"], case["dtype"],
                      shared_page=case["shared_page"])
    sg = torch.from_numpy(case["shared_gate"]) if case["shared_gate"] is not None else None
    y, w, ids = moe.forward(x, logits, case["k"], case["renorm"], shared_gate=sg)
    if case["Is"]:
        y_ref, w_ref, ids_ref = ref.fused_moe_shared_forward(
            case["x"], case["logits"], case["pool"], case["slot_map"], case["k"], case["renorm"],
            case["dtype"], shared_page=case["shared_page"], shared_gate_logits=case["shared_gate"])
    else:
        y_ref, w_ref, ids_ref = ref.fused_moe_forward(case["x"], case["logits"], case["pool"],
                                                      case["slot_map"], case["k"], case["renorm"],
                                                      case["dtype"])
    np.testing.assert_array_equal(ids.numpy(), ids_ref)
    np.testing.assert_allclose(w.numpy(), w_ref, rtol=1e-6, atol=0)
    return parity(y.numpy(), y_ref, TOL_BY_NAME[case["dtype"]], case=f"torch_cpu vs oracle {name}")


@pytest.mark.parametrize("name", ["c1_t32", "dsv2lite_t1", "qwen15_t4"])
def test_torch_cpu_baseline_matches_oracle(name):
    rec = _check(make_case(name), name)
    print(rec)


def test_torch_cpu_baseline_ties_and_small_bf16():
    """Equal logits pick the lowest expert indices; a small bf16 layer agrees with the oracle."""
    w, ids = TorchCpuMoE.route(torch.zeros((3, 8)), 2, True)
    assert ids.tolist() == [[0, 1]] * 3
    assert torch.equal(w, torch.full((3, 2), 0.5))
    rng = np.random.default_rng(5)
    T, H, I, E, k = 9, 128, 256, 8, 3
    pool = ref.f32_to_bf16_bits((rng.standard_normal((E, 3 * I * H)) * 0.05).astype(np.float32))
    x = ref.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    logits = ref.round_to(rng.standard_normal((T, E)).astype(np.float32), "bf16")
    case = dict(x=x, logits=logits, pool=pool, slot_map=np.arange(E), H=H, k=k, renorm=True,
                dtype="bf16", Is=0, shared_page=None, shared_gate=None)
    _check(case, "small")


def _mkl_check(case, name):
    from oracle import cpu_mkl
    if not cpu_mkl.available():
        pytest.skip("libmkl_rt is not installed")
    tc = TorchCpuMoE(case["pool"], case["slot_map"], case["H"], case["dtype"])
    I = next(iter(tc.w1.values())).shape[0]
    moe = cpu_mkl.MklCpuMoE(tc.w1, tc.w3, tc.w2, len(np.asarray(case["slot_map"]).reshape(-1)),
                            case["H"], I, case["dtype"], threads=4)
    x = ref.to_f32(case["x"], case["dtype"])
    y, w, ids = moe.forward(x, np.asarray(case["logits"], np.float32), case["k"], case["renorm"])
    y_ref, w_ref, ids_ref = ref.fused_moe_forward(case["x"], case["logits"], case["pool"],
                                                  case["slot_map"], case["k"], case["renorm"],
                                                  case["dtype"])
    np.testing.assert_array_equal(ids, ids_ref)
    np.testing.assert_allclose(w, w_ref, rtol=1e-6, atol=0)
    return parity(y, y_ref, TOL_BY_NAME[case["dtype"]], case=f"cpu_moe.cpp vs oracle {name}")


def test_cpp_mkl_baseline_matches_oracle():
    """oracle/cpu_moe.cpp (cblas_sgemm per expert, OpenMP) computes the oracle's layer: the
    reference's fp32 CPU configuration C1 (through its non-identity slot map) and a small bf16
    layer with an unmapped expert."""
    print(_mkl_check(make_case("c1_t32"), "c1_t32"))
    rng = np.random.default_rng(6)
    T, H, I, E, k = 21, 256, 128, 8, 2
    pool = ref.f32_to_bf16_bits((rng.standard_normal((E + 1, 3 * I * H)) * 0.05).astype(np.float32))
    slot_map = np.array([3, 0, 8, 1, 2, 7, -1, 5])  # expert 6 has no page: contributes nothing
    x = ref.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    logits = ref.round_to(rng.standard_normal((T, E)).astype(np.float32) * 2, "bf16")
    case = dict(x=x, logits=logits, pool=pool, slot_map=slot_map, H=H, k=k, renorm=False,
                dtype="bf16")
    print(_mkl_check(case, "small bf16"))
