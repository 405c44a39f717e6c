"""GPU producer parity: the synthetic generator and the codebook quantiser, bit-exact against the
reference's own outputs (golden fixtures written by the compiled reference) and the oracle."""
import hashlib
import json
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def ax():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import affinity_amd.experts as ax
    ax.init()
    return ax


def test_generator_matches_oracle(ax, orc):
    n = 1 << 22
    for seed, scale in ((1000, 0.02), (7, 1.0)):
        got = ax.gen_normal(seed, n, scale).cpu().numpy()
        ref = orc.normal_bf16(seed, n, scale)
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("case", ["a", "b", "c", "d"])
def test_quantizer_matches_reference_small(ax, small, c1_codebook, case):
    cbf = torch.from_numpy(ax.codebook_floats(c1_codebook)).cuda()
    w = small[f"{case}_w"]
    gw = torch.from_numpy(w).cuda()
    codes, fields, rs = ax.quantize_matrix(gw, cbf)
    np.testing.assert_array_equal(codes.cpu().numpy(), small[f"{case}_codes"])
    np.testing.assert_array_equal(fields.cpu().numpy(), small[f"{case}_fields"])
    np.testing.assert_array_equal(rs.cpu().numpy().view(np.uint16), small[f"{case}_rs"])
    imp = torch.from_numpy(small[f"{case}_imp"]).cuda()
    codes, fields, _ = ax.quantize_matrix(gw, cbf, imp)
    np.testing.assert_array_equal(codes.cpu().numpy(), small[f"{case}_codes_imp"])
    np.testing.assert_array_equal(fields.cpu().numpy(), small[f"{case}_fields_imp"])


def test_quantizer_matches_reference_config1(ax, c1_codebook):
    """The config-1 expert quantised on the GPU has the reference's exact plane hashes."""
    man = json.load(open(os.path.join(GOLDEN, "c1_manifest.json")))
    cbf = torch.from_numpy(ax.codebook_floats(c1_codebook)).cuda()
    H, I = 4096, 2048
    for m, (name, rows, cols) in enumerate((("gate", I, H), ("up", I, H), ("down", H, I))):
        w = ax.gen_normal(1000 + m, rows * cols, 0.02).view(rows, cols)
        assert sha(w.cpu().numpy()) == man["inputs"][name]
        codes, fields, rs = ax.quantize_matrix(w, cbf)
        torch.cuda.synchronize()
        assert sha(codes.cpu().numpy()) == man["planes"][name]["codes"], name
        assert sha(fields.cpu().numpy()) == man["planes"][name]["fields"], name
        assert sha(rs.cpu().numpy().view(np.uint16)) == man["planes"][name]["rscales"], name
