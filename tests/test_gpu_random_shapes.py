"""Seeded random shapes through the decode/verify and prefill paths against
the oracle: batch size, lengths (0, 1, page and tile edges included), GQA,
head_dim, page size, q_len 1..4, explicit or device-chosen partitions,
f32/bf16 q (the bf16 query takes the f16 QK with 16 or 32 rows per kv head
and in the prefill), appended rows; prefill causal ranges whole, split into
forced segments or split by the automatic plan.  Each case is fixed by its seed, so a failure
names a reproducible shape.  Bars as in test_gpu_parity.py."""
import math

import numpy as np
import pytest

from tests.test_gpu_parity import ATOL, RTOL, Scene, _bind_ctx, _run_decode, assert_close  # noqa: F401

pytestmark = pytest.mark.gpu


def _shape(seed):
    rng = np.random.default_rng(1000 + seed)
    D = int(rng.choice([128, 256]))
    PT = int(rng.choice([16, 32, 64, 128, 256]))
    Hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.choice([1, 2, 4, 8]))
    q_len = int(rng.choice([1, 1, 2, 4]))
    while q_len * G > 32:
        G //= 2
    B = int(rng.integers(1, 12))
    edges = [0, 1, PT - 1, PT, PT + 1, 31, 32, 33]
    lens = [int(rng.choice(edges)) if rng.random() < 0.3 else int(rng.integers(1, 1500))
            for _ in range(B)]
    lens = [max(L, q_len) for L in lens]
    part = 0 if rng.random() < 0.5 else int(max(32, PT) * rng.integers(1, 9))
    part = min(part, 64 * PT)
    return dict(D=D, PT=PT, Hkv=Hkv, Hq=Hkv * G, q_len=q_len, lens=lens, part=part,
                q_bf16=bool(rng.random() < 0.5), outliers=0.01 if rng.random() < 0.3 else 0.0)


@pytest.mark.parametrize("seed", range(24))
def test_random_decode_shapes(rkv, rko, ctx, seed):
    c = _shape(seed)
    print(f"seed {seed}: {c}", flush=True)
    sc = Scene(rkv, rko, c["Hkv"], c["D"], c["PT"], c["lens"], seed=seed, outliers=c["outliers"],
               src_bf16=True)
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((len(c["lens"]), c["q_len"], c["Hq"], c["D"])).astype(np.float32)
    if c["q_bf16"]:
        q = rko.bf16_to_f32(rko.f32_to_bf16(q)).reshape(q.shape)
    scale = 1.0 / math.sqrt(c["D"])
    got, pt = _run_decode(rkv, ctx, sc, q, scale, q_bf16=c["q_bf16"], q_len=c["q_len"],
                          partition_tokens=c["part"])
    want = rko.paged_decode(sc.lay, sc.pages, sc.bt, sc.lens,
                            np.arange(len(c["lens"]), dtype=np.int32), q, scale, pt)
    assert_close(got, want, what=f"seed {seed}")


@pytest.mark.parametrize("seed", range(8))
def test_random_prefill_shapes(rkv, rko, ctx, seed):
    torch = __import__("torch")
    rng = np.random.default_rng(2000 + seed)
    D = int(rng.choice([128, 256]))
    PT = int(rng.choice([16, 32, 64, 128, 256]))
    Hkv = int(rng.choice([1, 2]))
    G = int(rng.choice([1, 2, 4, 8, 16]))
    Hq = Hkv * G
    n_ent = int(rng.integers(1, 5))
    ents = [(int(rng.integers(0, 600)), int(rng.integers(1, 200))) for _ in range(n_ent)]
    print(f"seed {seed}: D={D} PT={PT} Hkv={Hkv} Hq={Hq} entries={ents}", flush=True)  # q dtype below
    lens = [c + n for c, n in ents]
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=seed, src_bf16=True)
    total = sum(n for _, n in ents)
    q = rng.standard_normal((total, Hq, D)).astype(np.float32)
    # drawn last so the shapes above stay those of the f32-only cases
    q_bf16 = bool(rng.random() < 0.5)
    if q_bf16:
        q = rko.bf16_to_f32(rko.f32_to_bf16(q)).reshape(q.shape)
    qd = torch.from_numpy(q).cuda()
    if q_bf16:
        qd = qd.to(torch.bfloat16)
    out = torch.full((total, Hq, D), float("nan"), device="cuda")
    a = rkv.prefill_args(list(range(n_ent)), [c for c, _ in ents], [n for _, n in ents], qd, out,
                         1.0 / math.sqrt(D))
    rkv.prefill_q8(ctx, sc.g, sc.pages_d, sc.bt_d, n_ent, a)
    ctx.sync()
    got = out.cpu().numpy()
    off = 0
    for i, (c, n) in enumerate(ents):
        L = np.array(sc.lens, np.int32).copy()
        L[i] = c + n
        want = rko.paged_decode(sc.lay, sc.pages, sc.bt, L, np.array([i], np.int32),
                                q[None, off:off + n], 1.0 / math.sqrt(D), 1024)[0]
        assert_close(got[off:off + n], want, what=f"seed {seed} entry {i}")
        off += n


@pytest.mark.parametrize("seed", range(8))
def test_random_prefill_split_shapes(rkv, rko, ctx, seed):
    """Prefill with contexts up to 2000 tokens and the causal ranges split
    into forced segments (or the automatic plan, or no workspace), mostly with
    a bf16 query: the pipelined tile loop over whole, partial and empty
    segments."""
    from tests import test_gpu_prefill as P
    rng = np.random.default_rng(5000 + seed)
    D = int(rng.choice([128, 256]))
    PT = int(rng.choice([16, 32, 64, 128, 256]))
    Hkv = int(rng.choice([1, 2]))
    G = int(rng.choice([1, 2, 4, 8, 16]))
    n_ent = int(rng.integers(1, 4))
    ents = [(int(rng.integers(0, 2000)), int(rng.integers(1, 150))) for _ in range(n_ent)]
    seg = [None, 0, int(max(32, PT) * rng.integers(1, 6))][int(rng.integers(0, 3))]
    q_bf16 = bool(rng.random() < 0.7)
    print(f"seed {seed}: D={D} PT={PT} Hkv={Hkv} G={G} entries={ents} segment={seg} bf16 q={q_bf16}",
          flush=True)
    lens = [c + n + int(rng.integers(0, 3)) for c, n in ents]
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=seed, src_bf16=True)
    ent = [(i, c, n) for i, (c, n) in enumerate(ents)]
    P._run(rkv, rko, ctx, sc, ent, Hkv * G, 1.0 / math.sqrt(D), q_bf16=q_bf16, seed=seed,
           segment_tokens=seg)


@pytest.mark.parametrize("seed", range(12))
def test_random_odd_group_shapes(rkv, rko, ctx, seed):
    """GQA groups that are not powers of two (3, 5, 6, 7, 12 q heads per kv
    head, so 3..28 rows per kv head with dead MFMA columns), a softmax scale
    of random sign and magnitude, then a prefill over the same pages with the
    same group (f32 or bf16 query, with or without the split workspace)."""
    from tests import test_gpu_prefill as P
    rng = np.random.default_rng(7000 + seed)
    D = int(rng.choice([128, 256]))
    PT = int(rng.choice([16, 32, 64, 128]))
    Hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.choice([3, 5, 6, 7, 12]))
    q_len = int(rng.choice([1, 2, 4]))
    while q_len * G > 32:
        q_len //= 2
    B = int(rng.integers(1, 8))
    lens = [max(int(rng.integers(1, 1200)), q_len) for _ in range(B)]
    scale = float(rng.choice([-1.0, 1.0]) * rng.uniform(0.25, 2.0) / math.sqrt(D))
    q_bf16 = bool(rng.random() < 0.5)
    part = 0 if rng.random() < 0.5 else int(max(32, PT) * rng.integers(1, 5))
    print(f"seed {seed}: D={D} PT={PT} Hkv={Hkv} G={G} q_len={q_len} lens={lens} scale={scale:+.4f} "
          f"bf16 q={q_bf16} part={part}", flush=True)
    sc = Scene(rkv, rko, Hkv, D, PT, lens, seed=seed, outliers=0.01, src_bf16=True)
    q = rng.standard_normal((B, q_len, Hkv * G, D)).astype(np.float32)
    if q_bf16:
        q = rko.bf16_to_f32(rko.f32_to_bf16(q)).reshape(q.shape)
    got, pt = _run_decode(rkv, ctx, sc, q, scale, q_bf16=q_bf16, q_len=q_len, partition_tokens=part)
    want = rko.paged_decode(sc.lay, sc.pages, sc.bt, sc.lens, np.arange(B, dtype=np.int32), q,
                            scale, pt)
    assert_close(got, want, what=f"seed {seed} decode")
    # prefill: each entry's last rows as a chunk after the rest of it
    ents = []
    for i, L in enumerate(lens):
        n = int(rng.integers(1, min(L, 40) + 1))
        ents.append((i, L - n, n))
    seg = [None, 0][int(rng.integers(0, 2))]
    P._run(rkv, rko, ctx, sc, ents, Hkv * G, scale, q_bf16=q_bf16, seed=seed, segment_tokens=seg)
