"""BASELINE config 4 (the mixed W4A4 / W8A8 MMDiT linear stack): one seeded block of 14 linears
through the drop-in ops against the oracle (rel-L2 < 4e-3 on sampled rows), and the assignment
and op count of the full 60-block stack."""
import numpy as np
import pytest
import torch

from kitchen_amd import synth
from oracle import gemm, linear, quant

pytestmark = pytest.mark.gpu


def test_stack_assignment_and_ops(gpu_device):
    print("[stack] 60-block assignment", flush=True)
    layers = synth.mmdit_linear_stack(blocks=60, device=gpu_device)
    assert len(layers) == 60 * 14
    # config 4's mix: exactly 35 % of the 840 linears on W4A4
    assert sum(l["fmt"] == "w4a4" for l in layers) == 294 == synth.w4a4_count(840)
    assert synth.stack_ops(layers) == pytest.approx(5.9155e13, rel=1e-4)
    del layers
    torch.cuda.empty_cache()


def test_one_block_against_oracle(gpu_device):
    layers = synth.mmdit_linear_stack(blocks=1, device=gpu_device)
    acts = synth.stack_activations(gpu_device)
    assert {l["fmt"] for l in layers} == {"w4a4", "w8a8"}
    for layer in layers:
        m, k, n = layer["M"], layer["K"], layer["N"]
        print(f"[stack] {layer['name']} {layer['fmt']} M={m} K={k} N={n}", flush=True)
        x = acts[(m, k)]
        y = synth.stack_layer(layer, x)
        torch.cuda.synchronize()
        rows = np.r_[0:32, m - 32:m] if m > 64 else np.arange(m)
        xf = x.float().cpu().numpy()[rows]
        t = {kk: v.cpu() for kk, v in layer["tensors"].items()}
        bias = t["bias"].float().numpy()
        if layer["fmt"] == "w4a4":
            qa, sa = quant.rotquant(xf, 64, 4)
            p = gemm.partials(qa, quant.unpack_i4(t["qweight"].numpy()), 64)
            ref = gemm.epilogue_group(p, sa, t["wscales"].numpy().astype(np.float64), bias)
        else:
            w = t["weight"].numpy()
            if w.ndim == 4:   # 16-row tiles [N/16, K/64, 16, 64] back to rows
                w = w.transpose(0, 2, 1, 3).reshape(-1, k)[:n]
            ref = linear.w8a8_linear(xf, w, t["weight_scale"].numpy(), bias, 256).y
        err = gemm.rel_l2(ref, y.float().cpu().numpy()[rows])
        assert err < 4e-3, (layer["name"], err)


def test_graph_replay_matches_eager(gpu_device):
    # one block captured in a HIP graph, replayed several times with eager work and syncs in
    # between; every replay's outputs equal the eager outputs bit for bit
    print("[stack] graph capture of one block", flush=True)
    layers = synth.mmdit_linear_stack(blocks=1, device=gpu_device)
    acts = synth.stack_activations(gpu_device)
    eager = [synth.stack_layer(l, acts[(l["M"], l["K"])]).clone() for l in layers]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for l in layers:
            synth.stack_layer(l, acts[(l["M"], l["K"])])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [synth.stack_layer(l, acts[(l["M"], l["K"])]) for l in layers]
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for l, y, ref in zip(layers, outs, eager):
            assert torch.equal(y, ref), (rep, l["name"])
        synth.stack_layer(layers[0], acts[(layers[0]["M"], layers[0]["K"])])   # eager work between replays
        torch.cuda.synchronize()


def test_dual_stream_graph_matches_single_stream(gpu_device):
    # two blocks: text linears on a side stream (joined after q/k/v and at each block end),
    # captured in one graph and replayed several times; outputs equal the single-stream pass
    print("[stack] dual-stream graph of two blocks", flush=True)
    layers = synth.mmdit_linear_stack(blocks=2, device=gpu_device)
    acts = synth.stack_activations(gpu_device)
    ref = [y.clone() for y in synth.stack_pass(layers, acts)]
    side = torch.cuda.Stream()
    warm = torch.cuda.Stream()
    warm.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(warm):
        eager2 = synth.stack_pass(layers, acts, side=side)
    torch.cuda.current_stream().wait_stream(warm)
    torch.cuda.synchronize()
    for l, y, r in zip(layers, eager2, ref):
        assert torch.equal(y, r), ("eager dual", l["name"])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = synth.stack_pass(layers, acts, side=side)
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for l, y, r in zip(layers, outs, ref):
            assert torch.equal(y, r), (rep, l["name"])
        synth.stack_layer(layers[1], acts[(layers[1]["M"], layers[1]["K"])])   # eager work between replays
        torch.cuda.synchronize()
