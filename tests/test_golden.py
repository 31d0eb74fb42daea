"""Golden fixtures (tests/golden/linear_small.npz, written by tests/golden/make_golden.py from the
oracle): the oracle still reproduces them (CPU), and the HIP kernels match them (GPU, C ABI)."""
import os

import numpy as np
import pytest
import torch

from conftest import REPO

GOLDEN = os.path.join(REPO, "tests", "golden", "linear_small.npz")


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_oracle_reproduces_golden(golden):
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(REPO, "tests", "golden", "make_golden.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    fresh = mod.build()
    assert set(fresh) == set(golden)
    for k, v in fresh.items():
        assert np.array_equal(np.asarray(v), golden[k]), k


def test_golden_fixture_shapes(golden):
    assert str(golden["spec"]) == "mq-oracle-1"
    assert golden["w4a8_partials"].shape == (4, 8, 16)
    assert golden["rq_h256_b8_q"].dtype == np.int8 and golden["rq_h256_b8_s"].dtype == np.float32
    assert (golden["rq_h0_b8_q"][1] == 0).all() and golden["rq_h0_b8_s"][1] == np.float32(1e-10)


@pytest.mark.gpu
def test_kernels_match_golden(golden, gpu_device):
    import kitchen_amd as ck
    from kitchen_amd import ops, synth
    from oracle import gemm

    print("[golden] rotquant + GEMM partials + linears", flush=True)
    x = synth.to_bf16_tensor(golden["x_bf16"], gpu_device)
    for key in [k[:-2] for k in golden if k.startswith("rq_") and k.endswith("_q")]:
        hb, bits = int(key.split("_")[1][1:]), int(key.split("_")[2][1:])
        q, s = ops.rotate_quantize(x, hb, bits)
        torch.cuda.synchronize()
        assert np.array_equal(q.cpu().numpy(), golden[key + "_q"]), key
        assert np.array_equal(s.cpu().numpy().view(np.uint32), golden[key + "_s"].view(np.uint32)), key
    qa, sa = ops.rotate_quantize(x, 256, 8)
    n = golden["w"].shape[0]
    qw = torch.from_numpy(golden["w4a8_q_packed"]).to(gpu_device)
    zp = torch.from_numpy(golden["w4a8_z_packed"]).to(gpu_device)
    part = ops.gemm_w4_group_partials(qa, qw, zp, n)
    torch.cuda.synchronize()
    assert np.array_equal(part.cpu().numpy(), golden["w4a8_partials"])
    y = ck.w4a8_int8_linear(x, qw, torch.from_numpy(golden["w4a8_s16"]).to(gpu_device), None, None, zp,
                            torch.from_numpy(golden["bias"]).to(gpu_device), 64, 256, torch.bfloat16)
    assert gemm.rel_l2(golden["w4a8_y"], y.float().cpu().numpy()) < 4e-3
    # device-side weight quantizer reproduces the fixture's codes
    qd, s16, zd = ck.quantize_w4a8_asym_weight(torch.from_numpy(golden["w"]).to(gpu_device), 64, 256)
    assert np.array_equal(qd.cpu().numpy(), golden["w4a8_q_packed"])
    assert np.array_equal(s16.cpu().numpy(), golden["w4a8_s16"]) and np.array_equal(zd.cpu().numpy(), golden["w4a8_z_packed"])
    y4 = ck.convrot_w4a4_linear(x, torch.from_numpy(golden["w4a4_q_packed"]).to(gpu_device),
                                torch.from_numpy(golden["w4a4_s16"]).to(gpu_device),
                                torch.from_numpy(golden["bias"]).to(gpu_device), convrot_groupsize=64)
    assert gemm.rel_l2(golden["w4a4_y"], y4.float().cpu().numpy()) < 4e-3
