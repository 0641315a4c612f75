"""Many tokens through one packed matrix (int8 MFMA) vs the decode dot.

The reference's prefill is the decode step per token (src/lib/tlm_model.c:
1105-1113), so every (token, row) output must carry the decode kernel's bits:
the token-batched kernel is checked bit for bit against the packed GEMV run
token by token (itself bit-exact with the oracle, test_hip_gemv.py), and a
sample against the oracle directly.  Shapes cover token counts around the
32-token tile, rows around the 16-row tile and the 128-row group, the edge
weight patterns of the reference's matvec tests, and poisoned activations,
for each weight format with a token kernel (Q4_K, Q5_K, Q6_K against Q8_K
activations; Q8_0 against a8 activations, eight blocks per staged 256
values)."""
import numpy as np
import pytest
import torch

import oracle
from tests.synth import random_code_rows
from tests.test_hip_gemv import make_wrow, same

pytestmark = pytest.mark.gpu


def run_case(hip, dev, dt, rows, n, ntok, seed, wmode=None, poison=False):
    rng = np.random.default_rng(seed)
    if wmode is None:
        W = random_code_rows(rng, dt, rows, n)
    else:
        W = np.stack([make_wrow(rng, dt, n, wmode if wmode >= 0 else int(rng.integers(0, 5))) for _ in range(rows)])
    rb = W.shape[1]
    X = (rng.standard_normal((ntok, n)) * rng.choice([0.1, 1.0, 30.0], size=(ntok, 1))).astype(np.float32)
    if poison and ntok > 3:
        X[1] = 0.0
        X[2, 5] = np.nan
        X[3, n - 1] = np.inf
    Wd = torch.from_numpy(W.reshape(-1)).to(dev)
    Wp = hip.pack(dt, Wd, rb, rows, n)
    kind = oracle.Q8_0 if dt == oracle.Q8_0 else oracle.Q8_K
    act = hip.quantize_act(kind, torch.from_numpy(X.reshape(-1)).to(dev))
    Y = hip.matmul_tokens(dt, Wp, rows, n, act, ntok)
    ab = oracle.qact_bytes(kind, n)
    want = torch.empty((ntok, rows), dtype=torch.float32, device=dev)
    for t in range(ntok):
        hip.matvec_packed(dt, Wp, rows, n, act[t * ab:(t + 1) * ab], want[t])
    torch.cuda.synchronize()
    got, want = Y.cpu().numpy(), want.cpu().numpy()
    ok = same(got, want)
    assert ok.all(), f"{(~ok).sum()} of {ok.size} outputs differ; first at {np.argwhere(~ok)[0]}"
    return W, X, got


KQ = [oracle.Q4_K, oracle.Q5_K, oracle.Q6_K, oracle.Q8_0]


@pytest.mark.parametrize("dt", KQ)
@pytest.mark.parametrize("rows,n,ntok", [(768, 2048, 32), (768, 2048, 1), (100, 512, 33), (2048, 768, 45),
                                         (130, 256, 64), (16, 256, 7), (768, 2048, 512)])
def test_tokmm_matches_decode(hip, dev, dt, rows, n, ntok):
    run_case(hip, dev, dt, rows, n, ntok, seed=rows * 7 + ntok + dt)


@pytest.mark.parametrize("dt", KQ)
@pytest.mark.parametrize("wmode", [1, 2, 3, 4, -1])
def test_tokmm_edge_weights(hip, dev, dt, wmode):
    run_case(hip, dev, dt, 48, 512, 19, seed=100 + wmode, wmode=wmode)


@pytest.mark.parametrize("dt", KQ)
def test_tokmm_poisoned_tokens(hip, dev, dt):
    run_case(hip, dev, dt, 96, 1024, 40, seed=7, poison=True)


@pytest.mark.parametrize("dt", KQ)
def test_tokmm_vs_oracle(hip, dev, dt):
    W, X, got = run_case(hip, dev, dt, 64, 512, 9, seed=3, wmode=3)
    for t in range(X.shape[0]):
        act = oracle.quantize_act(oracle.Q8_0 if dt == oracle.Q8_0 else oracle.Q8_K, X[t])
        want = oracle.matvec_rows(dt, W, W.shape[1], act, 512, 0, 64)
        assert same(got[t], want).all(), t


def test_tokmm_rejects_bad_arguments(hip, dev):
    from tierlm_amd._lib import HipError
    Wp = torch.zeros(4096, dtype=torch.uint8, device=dev)
    act = torch.zeros(4096, dtype=torch.uint8, device=dev)
    with pytest.raises(HipError):
        hip.matmul_tokens(oracle.Q6_K, Wp, 16, 100, act, 2)      # n not a multiple of 256
    with pytest.raises(HipError):
        hip.matmul_tokens(oracle.Q8_K, Wp, 16, 256, act, 2)      # dtype without a token kernel
