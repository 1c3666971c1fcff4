"""Device parity of the routing around the ops (router, moe_scatter, moe_gather), through the C-ABI, against the CPU
oracle; and a whole MoE layer on the device (router -> scatter -> gate_up_down -> gather) against the oracle's chain.

Bars: router ids equal (ties to the lower id), weights within 2e-6 relative (f32 softmax on the device with expf and a
butterfly sum against the oracle's double); scatter outputs equal; gather equal to the bit (the same f32 product and
add per slot, ascending, on the device's own weights and rows); the layer within relative L2 4e-3 (the reference's
device criterion for chains, tests/ref/test_exl3ref.py:336-346)."""
import numpy as np
import pytest

from cases import Case, Dev, rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import exl3c4
    exl3c4.lib()
    return torch


def _router(torch, lg_t, top_k, renorm):
    import exl3c4
    n_tok = lg_t.shape[0]
    ids = torch.full((n_tok, top_k), -7, dtype=torch.int32, device="cuda")
    w = torch.full((n_tok, top_k), -7.0, dtype=torch.float32, device="cuda")
    assert exl3c4.router_topk(lg_t, top_k, renorm, ids, w) == 0
    torch.cuda.synchronize()
    return ids.cpu().numpy(), w.cpu().numpy()


@pytest.mark.parametrize("n_tok,n_expert,top_k", [(8, 512, 10), (2048, 512, 10), (5, 64, 8), (3, 100, 1)])
def test_router_matches_the_oracle(torch_cuda, n_tok, n_expert, top_k):
    import oracle
    torch = torch_cuda
    print(f"router {n_tok}x{n_expert} top {top_k}", flush=True)
    rng = np.random.default_rng(n_tok + n_expert)
    lg = rng.standard_normal((n_tok, n_expert)).astype(np.float32)
    lg[::3] = np.round(lg[::3] * 4) / 4                          # ties in a third of the rows
    for renorm in (True, False):
        ids, w = _router(torch, torch.from_numpy(lg).cuda(), top_k, renorm)
        ids_o, w_o = oracle.router_topk(lg, top_k, renorm)
        assert np.array_equal(ids, ids_o)
        assert np.allclose(w, w_o, rtol=2e-6, atol=0)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_router_reads_f16_and_bf16_logits(torch_cuda, dt):
    import oracle
    torch = torch_cuda
    rng = np.random.default_rng(11)
    lg = torch.from_numpy(rng.standard_normal((16, 512)).astype(np.float32))
    lg_t = lg.to(torch.float16 if dt == "f16" else torch.bfloat16).cuda()
    ids, w = _router(torch, lg_t, 10, True)
    ids_o, w_o = oracle.router_topk(lg_t.float().cpu().numpy(), 10, True)
    assert np.array_equal(ids, ids_o) and np.allclose(w, w_o, rtol=2e-6, atol=0)


def _scatter(torch, ids_np, n_expert, base=0):
    import exl3c4
    n_tok, top_k = ids_np.shape
    T = n_tok * top_k
    ids = torch.from_numpy(ids_np.astype(np.int32)).cuda()
    st = torch.full((T,), -7, dtype=torch.int32, device="cuda")
    off = torch.full((n_expert + 1,), -7, dtype=torch.int32, device="cuda")
    cnt = torch.full((n_expert,), -7, dtype=torch.int32, device="cuda")
    row_of = torch.full((T,), -7, dtype=torch.int32, device="cuda")
    assert exl3c4.moe_scatter(ids, n_expert, st, off, cnt, row_of, expert_base=base) == 0
    torch.cuda.synchronize()
    return [a.cpu().numpy() for a in (st, off, cnt, row_of)]


@pytest.mark.parametrize("n_tok,top_k,n_expert,base,kind", [
    (8, 10, 512, 0, "router"), (37, 4, 16, 3, "drops"), (2048, 10, 512, 0, "zipf"), (1, 1, 1, 0, "one"),
    (300, 8, 1024, 5, "drops"), (0, 4, 8, 0, "empty")])
def test_scatter_matches_the_oracle(torch_cuda, n_tok, top_k, n_expert, base, kind):
    import exl3c4_synth as syn
    import oracle
    torch = torch_cuda
    print(f"scatter {kind} {n_tok}x{top_k} over {n_expert}", flush=True)
    rng = np.random.default_rng(n_tok * 7 + n_expert)
    if kind == "zipf":
        ids, _ = syn.zipf_topk(rng, n_tok, n_expert, top_k)
    elif kind == "router":
        ids, _ = oracle.router_topk(rng.standard_normal((n_tok, n_expert)).astype(np.float32), top_k)
    else:
        ids = rng.integers(-2, n_expert + base + 2, (n_tok, top_k)).astype(np.int32)
    got = _scatter(torch, np.asarray(ids, np.int32).reshape(n_tok, top_k), n_expert, base)
    want = oracle.moe_scatter_full(np.asarray(ids, np.int32).reshape(n_tok, top_k), n_expert, base)
    for g, w_, name in zip(got, want, ("sorted_tok", "expert_offset", "expert_count", "row_of")):
        assert np.array_equal(g, w_), name


@pytest.mark.parametrize("n_tok,E,top_k", [(8, 512, 10), (16, 512, 10), (40, 512, 10), (16, 8, 4), (16, 1024, 64),
                                            (3, 1, 1), (16, 64, 64), (5, 100, 7)])
def test_router_topk_scatter_matches_the_oracle(torch_cuda, n_tok, E, top_k):
    """The fused entry (one workgroup up to 16 tokens, the two launches beyond) against the oracle's router then
    scatter: many pairs an expert (8 experts), the most experts and pairs one workgroup scatters (1024 and 16 x 64),
    one expert, top_k = n_expert, an n_expert off the powers of two."""
    import exl3c4
    import oracle
    torch = torch_cuda
    print(f"router_topk_scatter {n_tok} tokens, {E} experts, top_k {top_k}", flush=True)
    rng = np.random.default_rng(100 + n_tok)
    lg = rng.standard_normal((n_tok, E)).astype(np.float32)
    if n_tok > 1:
        lg[1] = np.round(lg[1] * 2) / 2                          # ties
    T = n_tok * top_k
    ids = torch.full((n_tok, top_k), -7, dtype=torch.int32, device="cuda")
    w = torch.full((n_tok, top_k), -7.0, dtype=torch.float32, device="cuda")
    st = torch.full((T,), -7, dtype=torch.int32, device="cuda")
    off = torch.full((E + 1,), -7, dtype=torch.int32, device="cuda")
    cnt = torch.full((E,), -7, dtype=torch.int32, device="cuda")
    row_of = torch.full((T,), -7, dtype=torch.int32, device="cuda")
    assert exl3c4.router_topk_scatter(torch.from_numpy(lg).cuda(), top_k, True, ids, w, st, off, cnt, row_of) == 0
    torch.cuda.synchronize()
    ids_o, w_o = oracle.router_topk(lg, top_k, True)
    assert np.array_equal(ids.cpu().numpy(), ids_o) and np.allclose(w.cpu().numpy(), w_o, rtol=2e-6, atol=0)
    want = oracle.moe_scatter_full(ids_o, E)
    for g, w_, name in zip((st, off, cnt, row_of), want, ("sorted_tok", "expert_offset", "expert_count", "row_of")):
        assert np.array_equal(g.cpu().numpy(), w_), name


@pytest.mark.parametrize("n_tok,E,top_k,dt", [(8, 512, 10, "f32"), (5, 100, 7, "f16"), (1, 64, 64, "bf16"),
                                               (9, 512, 10, "f32")])
def test_router_topk_scatter_routes_to_the_bit_of_the_router(torch_cuda, n_tok, E, top_k, dt):
    """router_topk_scatter's routing (one workgroup, a wave a token) against router_topk's (a wave a token, four a
    workgroup) on the same logits: ids and weights to the bit, f32, f16 and bf16 logits, ties included (half-step
    logits in a row)."""
    import exl3c4
    torch = torch_cuda
    rng = np.random.default_rng(300 + n_tok)
    lg = rng.standard_normal((n_tok, E)).astype(np.float32)
    lg[0] = np.round(lg[0] * 2) / 2
    lg_t = torch.from_numpy(lg).cuda()
    if dt != "f32":
        lg_t = lg_t.to(torch.float16 if dt == "f16" else torch.bfloat16)
    T = n_tok * top_k
    for renorm in (True, False):
        ids_r, w_r = _router(torch, lg_t, top_k, renorm)
        ids = torch.full((n_tok, top_k), -7, dtype=torch.int32, device="cuda")
        w = torch.full((n_tok, top_k), -7.0, dtype=torch.float32, device="cuda")
        st = torch.full((T,), -7, dtype=torch.int32, device="cuda")
        off = torch.full((E + 1,), -7, dtype=torch.int32, device="cuda")
        assert exl3c4.router_topk_scatter(lg_t, top_k, renorm, ids, w, st, off, None, None) == 0
        torch.cuda.synchronize()
        assert np.array_equal(ids.cpu().numpy(), ids_r)
        assert np.array_equal(w.cpu().numpy().view(np.uint32), w_r.view(np.uint32))


@pytest.mark.parametrize("y_bf16", [True, False])
def test_gather_is_bit_exact(torch_cuda, y_bf16):
    import exl3c4
    import oracle
    torch = torch_cuda
    rng = np.random.default_rng(12)
    n_tok, top_k, E, cols = 64, 10, 512, 2048
    ids, w = oracle.router_topk(rng.standard_normal((n_tok, E)).astype(np.float32), top_k)
    ids[5, 3] = -1                                               # a dropped slot
    st, off, cnt, row_of = oracle.moe_scatter_full(ids, E)
    T = n_tok * top_k
    y = rng.standard_normal((T, cols)).astype(np.float32)
    yb = (torch.from_numpy(y).to(torch.bfloat16) if y_bf16 else torch.from_numpy(y).half()).view(torch.int16)
    out = torch.full((n_tok, cols), 0x7E7E, dtype=torch.int16, device="cuda")
    wt, rt = torch.from_numpy(w).cuda(), torch.from_numpy(row_of).cuda()
    assert exl3c4.moe_gather(yb.cuda(), y_bf16, wt, rt, out) == 0
    torch.cuda.synchronize()
    want = oracle.moe_gather(yb.numpy().view(np.uint16), y_bf16, w, row_of, n_tok, top_k)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), want)


def test_a_whole_layer_on_the_device(torch_cuda):
    """router -> scatter -> gate_up_down -> gather on the device (one kernel for gate_up_down: T = 48 rows), against
    the oracle's router, scatter, gate_up_down and gather on the same logits and weights."""
    import exl3c4
    import oracle
    torch = torch_cuda
    n_tok, top_k, E = 8, 6, 24
    rng = np.random.default_rng(13)
    logits = rng.standard_normal((n_tok, E)).astype(np.float32)
    ids_o, w_o = oracle.router_topk(logits, top_k, True)
    case = Case(seed=55, n_tok=n_tok, top_k=top_k, n_expert=E, geoms=[(256, 128)], bits=4, cb="mul1",
                expert_ids=ids_o)
    dev = Dev(case)
    print("layer on the device", flush=True)
    T = n_tok * top_k
    ids = torch.empty((n_tok, top_k), dtype=torch.int32, device="cuda")
    w = torch.empty((n_tok, top_k), dtype=torch.float32, device="cuda")
    assert exl3c4.router_topk(torch.from_numpy(logits).cuda(), top_k, True, ids, w) == 0
    st = torch.empty((T,), dtype=torch.int32, device="cuda")
    off = torch.empty((E + 1,), dtype=torch.int32, device="cuda")
    row_of = torch.empty((T,), dtype=torch.int32, device="cuda")
    assert exl3c4.moe_scatter(ids, E, st, off, None, row_of) == 0
    torch.cuda.synchronize()
    assert np.array_equal(st.cpu().numpy(), case.sorted_tok) and np.array_equal(off.cpu().numpy(), case.off)
    dev.sorted_tok, dev.off = st, off                            # the device's own routing drives the op
    y = dev.gate_up_down()
    assert dev.status == 0
    out = torch.empty((n_tok, y.shape[1]), dtype=torch.int16, device="cuda")
    yt = torch.from_numpy(y.view(np.int16)).cuda()
    assert exl3c4.moe_gather(yt, True, w, row_of, out) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.float16).astype(np.float32)
    _, _, _, row_of_o = oracle.moe_scatter_full(ids_o, E)
    y_o = case.oracle_gate_up_down()
    want = oracle.moe_gather(y_o, True, w_o, row_of_o, n_tok, top_k).view(np.float16).astype(np.float32)
    assert rel_l2(got, want) <= 4e-3
