"""Serving-style use of the operator: concurrent calls on two streams (each
stream caches its own workspace) and HIP graph capture + replay (the call
allocates nothing and never synchronises, so it is capturable once warm).
Every result is compared bitwise with a plain eager call on the same inputs."""
import pytest
import torch

from _helpers import gpu_args, log, run_gpu

from flashinfer_amd import kernel
from flashinfer_amd import workloads as W

pytestmark = pytest.mark.gpu
H = 7168


def _bits(x):
    return x.view(torch.int16).cpu()


def test_two_streams_concurrently():
    log("test_two_streams_concurrently")
    wa, wb = W.standard("c1_t64"), W.standard("t256")
    ref_a, ref_b = run_gpu(wa), run_gpu(wb)
    args_a, args_b = gpu_args(wa), gpu_args(wb)
    out_a = torch.empty(wa.T, H, dtype=torch.bfloat16, device="cuda")
    out_b = torch.empty(wb.T, H, dtype=torch.bfloat16, device="cuda")
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for _ in range(3):
        with torch.cuda.stream(sa):
            kernel.run(*args_a, out_a)
        with torch.cuda.stream(sb):
            kernel.run(*args_b, out_b)
    torch.cuda.synchronize()
    assert torch.equal(_bits(out_a), _bits(ref_a))
    assert torch.equal(_bits(out_b), _bits(ref_b))


@pytest.mark.parametrize("name,other", [("c1_t64", "c0_t16"), ("c2_t1024_o0", "c2_t1024_o64")])
def test_graph_capture_and_replay(name, other):
    """Capture one call, then replay it on fresh inputs copied into the captured
    tensors; every replay must equal an eager call on the same inputs."""
    log(f"test_graph_capture_and_replay[{name}]")
    wl = W.standard(name)
    static = gpu_args(wl)
    out = torch.empty(wl.T, H, dtype=torch.bfloat16, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm up: code objects load outside the capture
        kernel.run(*static, out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        kernel.run(*static, out)
    torch.cuda.synchronize()

    # inputs of the same shape: the original tokens, then tokens of another
    # workload truncated/padded to T (routing and activations change)
    alt = W.standard(other)
    variants = [wl.tensors]
    t2 = {k: v for k, v in wl.tensors.items()}
    n = min(wl.T, alt.T)
    for key in ("routing_logits", "hidden_states"):
        x = wl.tensors[key].clone()
        x[:n] = alt.tensors[key][:n]
        t2[key] = x
    s2 = wl.tensors["hidden_states_scale"].clone()
    s2[:, :n] = alt.tensors["hidden_states_scale"][:, :n]
    t2["hidden_states_scale"] = s2
    variants.append(t2)
    variants.append(wl.tensors)
    for i, t in enumerate(variants):
        static[0].copy_(t["routing_logits"])
        static[2].copy_(t["hidden_states"])
        static[3].copy_(t["hidden_states_scale"])
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = torch.empty_like(out)
        kernel.run(*static, eager)  # the program's own eager work between replays
        torch.cuda.synchronize()
        log(f"  replay {i}: equal={torch.equal(_bits(got), _bits(eager))}")
        assert torch.isfinite(got.float()).all()
        assert torch.equal(_bits(got), _bits(eager))


def test_graph_replay_with_gemm1_choice_flipping():
    """A captured T=1024 call holds both GEMM1 launches; the sort chooses
    between them at each replay from that replay's routing. Replays whose
    routing bias makes the LDS tile win (the captured inputs), then the wide
    kernel (another bias: fewer rows per expert), then the tile again, each
    equal the eager call on the same inputs bit for bit, and the eager calls
    show the choice flipping."""
    from flashinfer_amd import _lib
    log("test_graph_replay_with_gemm1_choice_flipping")
    wl = W.standard("c2_t1024_o0")
    static = gpu_args(wl)
    out = torch.empty(wl.T, H, dtype=torch.bfloat16, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        kernel.run(*static, out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        kernel.run(*static, out)
    torch.cuda.synchronize()
    bias_tile = wl.tensors["routing_bias"]
    bias_wide = W.standard_tokens("t256", T=wl.T).tensors["routing_bias"]  # 8 extra 64-row tiles
    L = _lib.workspace_layout(wl.T)
    chosen = []
    for bias in (bias_tile, bias_wide, bias_tile):
        static[1].copy_(bias)
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = torch.empty_like(out)
        kernel.run(*static, eager)
        torch.cuda.synchronize()
        meta = kernel.last_workspace()[L.expert_off:L.expert_off + 320 * 4].view(torch.int32).cpu()
        chosen.append(int(meta[256]))
        assert torch.isfinite(got.float()).all()
        assert torch.equal(_bits(got), _bits(eager))
    assert chosen == [1, 0, 1], chosen


def test_two_threads_one_stream():
    """Two Python threads calling run on the same stream at once each get
    their own workspace, so interleaved kernels of the two calls cannot mix
    tables: every output equals the single-threaded one bit for bit."""
    import threading
    log("test_two_threads_one_stream")
    wls = [W.standard("c1_t16"), W.standard("c1_t64")]
    refs = [run_gpu(wl).clone() for wl in wls]
    errors = []

    def worker(i):
        try:
            args = gpu_args(wls[i])
            out = torch.empty_like(refs[i])
            for _ in range(20):
                kernel.run(*args, out)
                torch.cuda.current_stream().synchronize()
                if not torch.equal(out.view(torch.int16), refs[i].view(torch.int16)):
                    errors.append(i)
                    return
        except Exception as exc:  # reported below
            errors.append(repr(exc))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors


def test_graphs_at_increasing_sizes_keep_their_workspaces():
    """Two graphs captured one after the other, the second at a larger T, then
    replayed in the opposite order and concurrently on two streams: each
    capture owns its workspace, so every replay equals an eager call on the
    same inputs (a shared, regrown workspace would leave the first graph
    writing into freed memory, and concurrent replays would mix tables)."""
    log("test_graphs_at_increasing_sizes_keep_their_workspaces")
    wls = [W.standard("c1_t16"), W.standard("c1_t64")]
    statics = [gpu_args(wl) for wl in wls]
    outs = [torch.empty(wl.T, H, dtype=torch.bfloat16, device="cuda") for wl in wls]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for st, o in zip(statics, outs):
            kernel.run(*st, o)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graphs = []
    for st, o in zip(statics, outs):  # T = 16, then T = 64 (a larger workspace)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            kernel.run(*st, o)
        graphs.append(g)
    torch.cuda.synchronize()
    refs = []
    for st, o in zip(statics, outs):
        e = torch.empty_like(o)
        kernel.run(*st, e)
        refs.append(e)
    torch.cuda.synchronize()
    for rep in range(3):
        for i in (1, 0):
            outs[i].fill_(float("nan"))
            graphs[i].replay()
            torch.cuda.synchronize()
            assert torch.equal(_bits(outs[i]), _bits(refs[i])), (rep, i)
            # eager work of the program between replays
            junk = torch.empty_like(outs[i])
            kernel.run(*statics[i], junk)
            torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for o in outs:
        o.fill_(float("nan"))
    torch.cuda.synchronize()
    for g, s in zip(graphs, streams):
        with torch.cuda.stream(s):
            g.replay()
    torch.cuda.synchronize()
    for i in range(2):
        assert torch.equal(_bits(outs[i]), _bits(refs[i])), ("concurrent", i)
    del graphs


def test_captured_workspaces_released_with_their_graphs():
    """Each captured call allocates its workspace from the graph's private
    pool and keeps no reference after the call: replays still equal eager
    calls, and destroying the graphs returns device memory to where it was
    before the captures."""
    import gc
    log("test_captured_workspaces_released_with_their_graphs")
    wls = [W.standard("c1_t16"), W.standard("c1_t64"), W.standard("t256")]
    statics = [gpu_args(wl) for wl in wls]
    outs = [torch.empty(wl.T, H, dtype=torch.bfloat16, device="cuda") for wl in wls]
    refs = [torch.empty_like(o) for o in outs]
    for st, r in zip(statics, refs):
        kernel.run(*st, r)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for st, o in zip(statics, outs):
            kernel.run(*st, o)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    gc.collect()
    base = torch.cuda.memory_allocated()
    graphs = []
    for st, o in zip(statics, outs):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            kernel.run(*st, o)
        graphs.append(g)
    torch.cuda.synchronize()
    held = torch.cuda.memory_allocated() - base
    for rep in range(3):
        for i, g in enumerate(graphs):
            outs[i].fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(_bits(outs[i]), _bits(refs[i])), (rep, i)
    del g, graphs
    gc.collect()
    torch.cuda.synchronize()
    after = torch.cuda.memory_allocated()
    log(f"  captured workspaces held {held / 2**20:.1f} MiB while the graphs lived; "
        f"after their release {(after - base) / 2**20:.1f} MiB")
    assert after <= base
