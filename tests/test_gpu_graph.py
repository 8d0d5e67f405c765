"""The decode step (append inside the launch, split-K decode, combine) captured
in HIP graphs, one per layer, as the long-context bench replays it: every
replay, with eager launches and synchronizations in between, must equal the
eager result bit for bit (the kernels are deterministic).  The captured
path records kernel launches only (no memset nodes)."""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _fill(rkv, ctx, pool, lens, Hkv, D, seed):
    import torch
    rng = np.random.default_rng(seed)
    for layer in range(pool.desc.layers):
        for s, L in enumerate(lens):
            k = torch.from_numpy(rng.standard_normal((L, Hkv, D)).astype(np.float32)).cuda()
            v = torch.from_numpy(rng.standard_normal((L, Hkv, D)).astype(np.float32)).cuda()
            pool.append(layer, torch.full((L,), s, dtype=torch.int32, device="cuda"),
                        torch.arange(L, dtype=torch.int32, device="cuda"), k, v)
    ctx.sync()


@pytest.mark.parametrize("lens,part", [([3000, 1500, 777, 65], 0), ([20000], 0), ([900, 5000], 1024)])
def test_decode_graph_replays_match_eager(rkv, ctx, lens, part):
    import torch
    Hq, Hkv, D, PT, layers = 16, 2, 256, 64, 2
    B = len(lens)
    W = max((L + PT - 1) // PT for L in lens)
    pool = rkv.Pool(ctx, layers, Hkv, D, PT, sum((L + PT - 1) // PT for L in lens) + 4, B, W, seed=5)
    for s, L in enumerate(lens):
        pool.alloc.reserve(s, L)
    pool.sync_tables()
    _fill(rkv, ctx, pool, lens, Hkv, D, seed=len(lens))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    seq_ids = torch.arange(B, dtype=torch.int32, device="cuda")
    pos = torch.tensor([L - 1 for L in lens], dtype=torch.int32, device="cuda")
    k_new = torch.randn((B, Hkv, D), generator=gen, device="cuda").to(torch.bfloat16)
    v_new = torch.randn((B, Hkv, D), generator=gen, device="cuda").to(torch.bfloat16)
    q = torch.randn((B, 1, Hq, D), generator=gen, device="cuda").to(torch.bfloat16)
    outs = [torch.empty((B, 1, Hq, D), dtype=torch.float32, device="cuda") for _ in range(layers)]
    app = rkv.append_args(seq_ids, pos, k_new, v_new)
    args = []
    for layer in range(layers):
        a = rkv.decode_args(q, outs[layer], seq_ids, 1.0 / math.sqrt(D), max(lens),
                            partition_tokens=part, append=app)
        ws = torch.empty(max(rkv.decode_workspace_bytes(pool.geometry, a), 4), dtype=torch.uint8,
                         device="cuda")
        a = rkv.decode_args(q, outs[layer], seq_ids, 1.0 / math.sqrt(D), max(lens),
                            partition_tokens=part, workspace=ws, append=app)
        a._ws = ws
        args.append(a)

    # eager reference (the appended rows are rewritten with the same bytes on
    # every launch, so every later launch sees the same cache)
    for layer in range(layers):
        pool.decode(layer, args[layer])
    ctx.sync()
    want = [o.clone() for o in outs]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for layer in range(layers):
            pool.decode(layer, args[layer], stream=side)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graphs = []
    for layer in range(layers):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            pool.decode(layer, args[layer], stream=torch.cuda.current_stream())
        graphs.append(g)
    torch.cuda.synchronize()

    scratch = torch.empty_like(outs[0])
    for rep in range(4):
        for layer in range(layers):
            outs[layer].fill_(float("nan"))
            # eager work between replays: the other layer's decode, eagerly
            other = rkv.decode_args(q, scratch, seq_ids, 1.0 / math.sqrt(D), max(lens),
                                    partition_tokens=part, workspace=args[1 - layer]._ws,
                                    append=app)
            pool.decode(1 - layer, other)
            torch.cuda.synchronize()
            graphs[layer].replay()
            torch.cuda.synchronize()
            assert torch.equal(outs[layer], want[layer]), f"replay {rep} layer {layer}"
            assert torch.equal(scratch, want[1 - layer]), f"eager between replays, rep {rep}"
    del graphs
    pool.close()
