"""The ops under HIP graph capture (torch.cuda.CUDAGraph): captured once, replayed several times with eager
work and synchronisations between the replays, every replay bit for bit equal to the eager call.

This covers the split-K counters at the head of the workspace, whose per-call tag is baked into the captured
kernel arguments: the last arrival of each tile clears its counter word, so every replay finds it empty (the
workspace contract in include/qk_abi.h). No op issues a memset or allocates inside the library, so nothing
else is captured but kernels.
"""
import pytest
import torch

from op_plugin_amd import workloads as W

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import op_plugin_amd
    return op_plugin_amd


def say(msg):
    print(f"[case] {msg}", flush=True)


def _inputs():
    g = torch.Generator().manual_seed(11)
    x = torch.randn((16, 4096), generator=g).to(torch.float16)
    w8 = torch.randint(-127, 128, (4096, 4096), generator=g, dtype=torch.int8)      # [K, N]
    s8 = (1e-3 + 9e-3 * torch.rand(4096, generator=g)).float()
    bias = (0.1 * torch.randn(4096, generator=g)).to(torch.bfloat16)
    c = W.W4A16Case(M=16, N=11008, K=4096, group=128, x_dtype=torch.bfloat16, offset=True)
    d4 = W.w4a16_inputs(c, seed=3)
    return dict(x=x.to(DEV), w8=w8.to(DEV), s8=s8.to(DEV), bias=bias.to(DEV), x4=d4["x"].to(DEV),
                w4=d4["w_packed"].to(DEV), sc4=d4["scale"].to(DEV), of4=d4["offset"].to(DEV))


def _path(ops, t, w4nz):
    """dynamic quant -> W8A8 (M = 16 on a [K,N] weight: the split stream + reduce), W4A16 decode on the
    row-major weight (split-K stream with its counters) and on the NZ weight."""
    xq, xs = ops.npu_dynamic_quant(t["x"])
    y8 = ops.npu_quant_matmul(xq, t["w8"], t["s8"], pertoken_scale=xs, bias=t["bias"], output_dtype=torch.bfloat16)
    y4 = ops.npu_weight_quant_batchmatmul(t["x4"], t["w4"], t["sc4"], t["of4"], antiquant_group_size=128)
    y4nz = ops.npu_weight_quant_batchmatmul(t["x4"], w4nz, t["sc4"], t["of4"], antiquant_group_size=128)
    return xq, xs, y8, y4, y4nz


def test_graph_replays_match_eager(ops):
    say("HIP graph: dynamic quant + W8A8 split stream + W4A16 split stream + NZ decode, 5 replays")
    t = _inputs()
    w4nz = ops.npu_format_cast(t["w4"], 29)
    eager = [r.clone() for r in _path(ops, t, w4nz)]
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _path(ops, t, w4nz)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = _path(ops, t, w4nz)
    torch.cuda.synchronize()

    for r in range(5):
        for o in captured:
            o.zero_()  # a fill kernel, not a memset node; the replay must rewrite every output
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, ref in zip(("y", "scale", "w8a8", "w4a16", "w4a16_nz"), captured, eager):
            assert torch.equal(got, ref), f"replay {r}: {name} differs from the eager call"
        # eager work between the replays, on the same workspace-holding allocator and stream
        again = _path(ops, t, w4nz)
        torch.cuda.synchronize()
        for name, got, ref in zip(("y", "scale", "w8a8", "w4a16", "w4a16_nz"), again, eager):
            assert torch.equal(got, ref), f"eager call after replay {r}: {name} differs"


def test_graph_replays_mlp_block(ops):
    """The cfg5 quantized MLP block on NZ weights under capture: RMSNorm + quant, the gate-up GEMM with the SwiGLU
    and the row absmax in its epilogue (h and the partials in a workspace the op takes from the allocator), the
    premax quantizer, and the down projection's 128-row K split (tagged counters, int32 partials, reduce)."""
    from op_plugin_amd.mlp import quant_mlp
    say("HIP graph: cfg5 MLP block (512 x 4096 x 14336) on NZ weights, 3 replays")
    g = torch.Generator(device=DEV).manual_seed(5)
    T, H, I = 512, 4096, 14336
    x = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
    gamma = (1 + 0.02 * torch.randn(H, generator=g, device=DEV)).to(torch.bfloat16)
    wgu = ops.npu_format_cast(torch.randint(-127, 128, (H, 2 * I), generator=g, device=DEV, dtype=torch.int8), 29)
    sgu = 1e-3 + 9e-3 * torch.rand(2 * I, generator=g, device=DEV)
    wd = ops.npu_format_cast(torch.randint(-127, 128, (I, H), generator=g, device=DEV, dtype=torch.int8), 29)
    sd = 1e-3 + 9e-3 * torch.rand(H, generator=g, device=DEV)

    def run():
        return quant_mlp(x, gamma, wgu, sgu, wd, sd)

    eager = run().clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = run()
    torch.cuda.synchronize()
    for r in range(3):
        captured.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"replay {r}: the block's output differs from the eager call"
        again = run()
        torch.cuda.synchronize()
        assert torch.equal(again, eager), f"eager call after replay {r} differs"


def test_graph_replays_nz_prefill_stream_k(ops):
    """The NZ prefill kernel's stream-K schedule under capture (cfg3's width, M = 1024: 344 tiles on one
    workgroup per CU): one tag per graph, so each replay must find the range-boundary counters cleared by the
    previous one's last arrivals, and read only partial slots written in the same replay."""
    from op_plugin_amd import workloads as W
    say("HIP graph: W4A16 NZ prefill, stream-K (1024 x 11008 x 4096), 3 replays")
    d = W.w4a16_inputs(W.W4A16Case(M=1024, N=11008, K=4096, group=128, x_dtype=torch.bfloat16, offset=True), seed=17)
    x, sc, off = d["x"].to(DEV), d["scale"].to(DEV), d["offset"].to(DEV)
    nz = ops.npu_format_cast(d["w_packed"].to(DEV), 29)

    def run():
        return ops.npu_weight_quant_batchmatmul(x, nz, sc, off, antiquant_group_size=128)

    eager = run().clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = run()
    torch.cuda.synchronize()
    for r in range(3):
        captured.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"replay {r}: the prefill output differs from the eager call"
        again = run()
        torch.cuda.synchronize()
        assert torch.equal(again, eager), f"eager call after replay {r} differs"
