"""GPU parity of the device router (affx_route_topk) against the oracle's restatement of the
engine's route_topk (itself pinned to the reference's outputs, tests/test_oracle.py) and of the
configs' softmax rule, and the router feeding the decode and grouped paths with no host round
trip."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import oracle_ffn_tokens, random_expert_container, rel_l2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ax():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import affinity_amd.experts as ax
    ax.init()
    return ax


def ulps(a: np.ndarray, b: np.ndarray) -> int:
    """Largest distance in units in the last place between two float32 arrays of one sign."""
    ai = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    return int(np.abs(ai - bi).max()) if a.size else 0


def _route(logits: torch.Tensor, k, rule, bias=None, norm=True, scaling=1.0, dim_major=False):
    from affinity_amd._lib import check, lib
    if dim_major:          # logits given as the engine's [n_expert][nb] arena
        n_expert, T = logits.shape
        ts, es = 1, logits.stride(0)
    else:
        T, n_expert = logits.shape
        ts, es = logits.stride(0), 1
    sel = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    check(lib().affx_route_topk(logits.data_ptr(), ts, es, 0 if bias is None else bias.data_ptr(), T, n_expert, k,
                                rule, int(norm), float(scaling), sel.data_ptr(), w.data_ptr(),
                                torch.cuda.current_stream().cuda_stream), "route_topk")
    return sel, w


@pytest.mark.parametrize("dim_major", [False, True])
def test_engine_rule_matches_oracle(ax, orc, dim_major):
    """route_topk on 2000 tokens x 256 experts (logit scales 0.3..6, a bias on every other run, a
    few logits past softplus's x > 20 guard): ids bit for bit; weights within 2 ulp (the device
    scores are within an ulp of the host's float expf/log1pf, which are not correctly rounded)."""
    from affinity_amd._lib import AFFX_ROUTE_ENGINE
    rng = np.random.default_rng(3 + dim_major)
    T, E, k = 2000, 256, 6
    lg = (rng.standard_normal((T, E)) * rng.uniform(0.3, 6, (T, 1))).astype(np.float32)
    lg[::97, 5] = 23.0
    for use_bias in (False, True):
        bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if use_bias else None
        gl = torch.from_numpy(lg.T.copy() if dim_major else lg).cuda()
        gb = None if bias is None else torch.from_numpy(bias).cuda()
        sel, w = _route(gl, k, AFFX_ROUTE_ENGINE, gb, True, 1.5, dim_major)
        sel, w = sel.cpu().numpy(), w.cpu().numpy()
        worst = 0
        for t in range(T):
            rs, rw = orc.route_topk(lg[t], bias, k, True, 1.5)
            np.testing.assert_array_equal(sel[t], rs, err_msg=f"token {t}")
            worst = max(worst, ulps(w[t], rw))
        print(f"engine rule (bias={use_bias}, dim_major={dim_major}): ids exact, weights within {worst} ulp")
        assert worst <= 2


def test_engine_rule_ties_floor_and_no_renorm(ax, orc):
    """Exact ties go to the lower id; all-negative logits hit the sum floor; without
    renormalisation the weight is score * scaling."""
    from affinity_amd._lib import AFFX_ROUTE_ENGINE
    rng = np.random.default_rng(9)
    E, k = 256, 8
    lg = rng.standard_normal((4, E)).astype(np.float32)
    lg[0, [200, 7, 99, 150, 3, 250, 31, 64, 128]] = 4.0       # nine tied at the top
    lg[1, :] = 1.25                                           # every expert tied
    lg[2, :] = -70.0                                          # scores ~1e-15: the sum floor
    for norm in (True, False):
        sel, w = _route(torch.from_numpy(lg).cuda(), k, AFFX_ROUTE_ENGINE, None, norm, 2.0)
        sel, w = sel.cpu().numpy(), w.cpu().numpy()
        for t in range(4):
            rs, rw = orc.route_topk(lg[t], None, k, norm, 2.0)
            np.testing.assert_array_equal(sel[t], rs)
            assert ulps(w[t], rw) <= 2
    assert list(sel[0]) == [3, 7, 31, 64, 99, 128, 150, 200] and list(sel[1]) == list(range(8))


def test_softmax_rule_matches_oracle(ax, orc):
    """The configs' rule: ids bit for bit against the oracle and against the torch form the bench
    uses; weights within 1 ulp."""
    from affinity_amd import synthetic
    from affinity_amd._lib import AFFX_ROUTE_SOFTMAX
    lg = ax.gen_normal(synthetic.S_R, 512 * 256, 1.0, bf16_round=False).view(512, 256)
    sel, w = _route(lg, 6, AFFX_ROUTE_SOFTMAX)
    ts, tw = synthetic.softmax_topk(lg, 6)
    assert torch.equal(sel, ts)
    assert ulps(w.cpu().numpy(), tw.cpu().numpy()) <= 1
    lgn = lg.cpu().numpy()
    for t in range(0, 512, 7):
        rs, rw = orc.route(lgn[t], 6)
        np.testing.assert_array_equal(sel[t].cpu().numpy(), rs)
        assert ulps(w[t].cpu().numpy(), rw) <= 1


def test_router_feeds_decode_and_grouped_without_host(ax, orc, c1_codebook):
    """Logits -> affx_route_topk -> affx_expert_ffn_decode (captured together in a HIP graph: no
    host round trip between them) and -> affx_expert_ffn_grouped, against the oracle run on the
    oracle's own routes."""
    from affinity_amd._lib import AFFX_ROUTE_ENGINE, check, lib
    hidden, inter, n = 2048, 1024, 32
    rng = np.random.default_rng(12)
    lay = ax.expert_layout(hidden, inter)
    ex = np.stack([random_expert_container(rng, hidden, inter, lay) for _ in range(n)])
    pool = ax.ExpertPool.from_container(torch.from_numpy(ex.reshape(-1)).cuda(), c1_codebook, hidden, inter)
    cbf = orc.unpack_codebook(c1_codebook)
    experts = {e: np.ascontiguousarray(ex[e]) for e in range(n)}
    bias = (rng.standard_normal(n) * 0.05).astype(np.float32)
    gb = torch.from_numpy(bias).cuda()

    def oracle_routes(lg):
        rs = [orc.route_topk(lg[t], bias, 6, True, 1.5) for t in range(lg.shape[0])]
        return np.stack([r[0] for r in rs]).astype(np.uint32), np.stack([r[1] for r in rs])

    # decode: M = 4 tokens, router and decode in one graph
    M = 4
    lg = rng.standard_normal((M, n)).astype(np.float32)
    x = (rng.standard_normal((M, hidden)) * 0.5).astype(np.float32)
    glg, gx = torch.from_numpy(lg).cuda(), torch.from_numpy(x).cuda()
    sel = torch.empty((M, 6), dtype=torch.int32, device="cuda")
    w = torch.empty((M, 6), device="cuda")
    y = torch.zeros((M, hidden), device="cuda")
    ws = ax.DecodeWorkspace(M, 6, hidden, inter)
    L = pool.layer()

    def step(stream):
        check(lib().affx_route_topk(glg.data_ptr(), n, 1, gb.data_ptr(), M, n, 6, AFFX_ROUTE_ENGINE, 1, 1.5,
                                    sel.data_ptr(), w.data_ptr(), stream), "route")
        check(lib().affx_expert_ffn_decode(C.byref(L), gx.data_ptr(), hidden, 1, M, sel.data_ptr(), w.data_ptr(), 6,
                                           y.data_ptr(), hidden, 1, 0, ws.buf.data_ptr(), ws.bytes, stream), "decode")

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(s.cuda_stream)
        torch.cuda.synchronize()
        eager = y.clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            step(s.cuda_stream)
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
    rs, rw = oracle_routes(lg)
    np.testing.assert_array_equal(sel.cpu().numpy(), rs)
    ref = oracle_ffn_tokens(orc, experts, cbf, x, rs, rw, range(M), hidden, inter)
    err = rel_l2(y.cpu().numpy(), ref)
    print(f"router -> decode (graph) rel_l2={err:.3e}")
    assert err <= 1e-3 and ws.status() == 0

    # grouped: 200 tokens
    T = 200
    lg = rng.standard_normal((T, n)).astype(np.float32)
    xb = torch.from_numpy(rng.standard_normal((T, hidden)).astype(np.float32)).cuda().to(torch.bfloat16)
    sel, w = _route(torch.from_numpy(lg).cuda(), 6, AFFX_ROUTE_ENGINE, gb, True, 1.5)
    yg = ax.expert_ffn_grouped(pool, xb, sel, w).cpu().numpy()
    rs, rw = oracle_routes(lg)
    np.testing.assert_array_equal(sel.cpu().numpy(), rs)
    ref = oracle_ffn_tokens(orc, experts, cbf, xb.float().cpu().numpy(), rs, rw, range(T), hidden, inter)
    err = rel_l2(yg, ref)
    print(f"router -> grouped rel_l2={err:.3e}")
    assert err <= 1e-3
