"""The ``gnn_amd::*`` torch operators on the GPU: torch.library.opcheck (schema, fake
implementation, no aliasing) and whole-graph capture by torch.compile (aot_eager backend,
no code generation) of a block that calls the public API, equal to eager bit for bit."""

import pytest
import torch

from helpers import attention_inputs, pair_input, trimul_weights

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _attn_args():
    t = attention_inputs(1, 3, 40, 2, 32, torch.bfloat16, seed=1)
    mask = torch.ones(1, 3, 1, 1, 40, dtype=torch.bool)
    mask[..., 33:] = False
    return tuple(x.to(DEV) for x in (t["q"], t["k"], t["v"], t["bias"], mask))


def _trimul_args():
    w = {k: v.to(DEV) for k, v in trimul_weights(64, 32, torch.bfloat16, seed=2, biases=True).items()}
    x, mask = pair_input(1, 24, 64, torch.bfloat16, seed=3)
    return x.to(DEV), mask.to(DEV), w


def test_opcheck_triangle_attention():
    import geometric_nn_ops_torch._ops  # noqa: F401  (registers the operators)

    q, k, v, bias, mask = _attn_args()
    torch.library.opcheck(torch.ops.gnn_amd.triangle_attention_fwd.default, (q, k, v, bias, mask, None),
                          test_utils=("test_schema", "test_faketensor"))


def test_opcheck_trimul():
    import geometric_nn_ops_torch._ops  # noqa: F401

    x, mask, w = _trimul_args()
    args = (x, "incoming", mask, w["norm_in_weight"], w["norm_in_bias"], w["p_in_weight"], w["p_in_bias"],
            w["g_in_weight"], w["g_in_bias"], w["norm_out_weight"], w["norm_out_bias"], w["p_out_weight"],
            w["p_out_bias"], w["g_out_weight"], w["g_out_bias"], 1e-5)
    torch.library.opcheck(torch.ops.gnn_amd.trimul_fwd.default, args,
                          test_utils=("test_schema", "test_faketensor"))


def test_compile_fullgraph_matches_eager():
    from geometric_nn_ops_torch.triangle import triangle_attention, triangle_multiplicative_update

    q, k, v, bias, amask = _attn_args()
    x, tmask, w = _trimul_args()

    def block(q, k, v, bias, amask, x, tmask):
        o = triangle_attention(q, k, v, bias, amask)
        y = triangle_multiplicative_update(x, "outgoing", tmask, **w)
        return o, y

    with torch.no_grad():
        eager = block(q, k, v, bias, amask, x, tmask)
        torch._dynamo.reset()
        compiled = torch.compile(block, fullgraph=True, backend="aot_eager")(q, k, v, bias, amask, x, tmask)
    for e, c in zip(eager, compiled):
        assert torch.equal(e, c)


def test_hip_graph_replays_match_eager():
    """The entry points are capturable: attention (with its bias pre-pass) and both trimul
    directions captured once as a HIP graph and replayed several times, with eager work and
    synchronisations between the replays; every replay equals the eager result bit for bit.
    (The library records no memset nodes: its scratch is rewritten in full by each call.)"""
    from geometric_nn_ops_torch.triangle import triangle_attention, triangle_multiplicative_update

    q, k, v, bias, amask = _attn_args()
    x, tmask, w = _trimul_args()

    def block():
        return (triangle_attention(q, k, v, bias, amask),
                triangle_multiplicative_update(x, "outgoing", tmask, **w),
                triangle_multiplicative_update(x, "incoming", tmask, **w))

    with torch.no_grad():
        eager = block()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm the allocator and the library off the capture
            block()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            captured = block()
        for replay in range(4):
            for t in captured:
                t.zero_()
            graph.replay()
            torch.cuda.synchronize()
            for got, want in zip(captured, eager):
                assert torch.equal(got, want), replay
            block()  # eager work between the replays
            torch.cuda.synchronize()
