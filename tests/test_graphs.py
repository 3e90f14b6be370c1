"""Every entry point under HIP graph capture: after one eager call (which allocates the op's
workspace), a call captured into a graph replays with the same bits as an eager call, on
input values that change between replays (scalar arguments are passed by value, so a
graph keeps the captured ones).  The calls record no memset node (workspaces are
zeroed by kernels) and allocate nothing, so capture succeeds; between replays the test
does its own eager work and synchronises, and checks every replay."""
import pytest
import torch

from cob_amd import capi, inputs

pytestmark = pytest.mark.gpu

SMALL = {
    "pow_abs_sqrt_mean": dict(name="g", seed=1, batch_size=2, height=33, width=65),
    "leaky": dict(name="g", seed=2, T=17, B=3, H=130, mem0_std=0.1),
    "reward_to_go": dict(name="g", seed=3, B=5, T=2100, gamma=0.95, done_p=0.05),
    "ppo_clip": dict(name="g", seed=4, B=300, T=31, H=2),
    "efficient_kan": dict(name="g", seed=5, B=300, I=64, O=96),
    "fp8_linear": dict(name="g", seed=6, M=300, K=256, N=264),
}


def _bind(op, inp):
    args = capi.device_args(op, inp)
    outs = {}
    if op == "ppo_clip":
        outs["output"] = torch.empty(6, device="cuda")
    else:
        for name, (shape, dtype) in capi.output_shapes(op, inp).items():
            outs[name] = torch.empty(shape, dtype=dtype, device="cuda")
    args.update(outs)
    return args, outs


@pytest.mark.parametrize("op", list(SMALL))
def test_graph_replay_matches_eager(lib, op):
    print(f"\n[graph] {op}", flush=True)
    case = SMALL[op]
    args, outs = _bind(op, inputs.make_inputs(op, case))
    capi.call(lib, op, args)           # eager call first: the workspace is allocated here
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        capi.call(lib, op, args)       # on the capture stream (torch's current stream)

    for k in range(3):
        new = inputs.make_inputs(op, case, case["seed"] + 100 + k)
        dev = capi.device_args(op, new)
        for name, t in dev.items():    # new values at the same pointers, written eagerly
            if isinstance(t, torch.Tensor):
                args[name].copy_(t)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = {n: t.clone() for n, t in outs.items()}
        # Scalar arguments (fp8_linear's scales, gamma, eps) are by value, so the graph
        # keeps the captured ones; the eager call uses the same.
        want_args, want_outs = _bind(op, new)
        want_args.update({k: v for k, v in args.items() if not isinstance(v, torch.Tensor)})
        capi.call(lib, op, want_args)
        torch.cuda.synchronize()
        for n in outs:
            assert torch.equal(got[n].reshape(-1).view(torch.uint8), want_outs[n].reshape(-1).view(torch.uint8)), (k, n)


def test_graph_of_several_ops(lib):
    """One graph holding a sequence of different ops (their workspaces all allocated first)."""
    ops = ["reward_to_go", "ppo_clip", "pow_abs_sqrt_mean", "fp8_linear"]
    bound = {op: _bind(op, inputs.make_inputs(op, SMALL[op])) for op in ops}
    for op, (args, _) in bound.items():
        capi.call(lib, op, args)
    torch.cuda.synchronize()
    want = {op: {n: t.clone() for n, t in outs.items()} for op, (_, outs) in bound.items()}
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for op, (args, _) in bound.items():
            capi.call(lib, op, args)
    for _ in range(3):
        for _, outs in bound.values():
            for t in outs.values():
                t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for op, (_, outs) in bound.items():
            for n, t in outs.items():
                assert torch.equal(t, want[op][n]), (op, n)
