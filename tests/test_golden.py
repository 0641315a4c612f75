"""Golden fixtures written by the compiled reference (tests/golden/gen_golden.py):
the oracle must reproduce them on the CPU, and the HIP path on the GPU."""
import os

import numpy as np
import pytest

import oracle
from oracle import Q4_K, Q5_K, Q6_K, Q8_0, Q8_K

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
INT = [Q8_0, Q4_K, Q5_K, Q6_K, Q8_K]


def load(name):
    return np.load(os.path.join(G, name))


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


def test_oracle_quantisers_match_golden():
    z = load("quant_rows.npz")
    for dt in INT:
        for n in (256, 512, 2048, 768):
            assert np.array_equal(oracle.quantize_row(dt, z[f"x_{dt}_{n}"]), z[f"q_{dt}_{n}"]), (dt, n)


def test_oracle_activations_match_golden():
    z = load("act.npz")
    i = 0
    while f"x{i}" in z:
        assert np.array_equal(oracle.quantize_act(Q8_K, z[f"x{i}"]), z[f"k{i}"]), i
        assert np.array_equal(oracle.quantize_act(Q8_0, z[f"x{i}"]), z[f"a{i}"]), i
        i += 1
    assert i >= 6


def test_oracle_dots_match_golden():
    z = load("dots.npz")
    for dt in INT:
        for n in (256, 768, 2048):
            W, act, y = z[f"w_{dt}_{n}"], z[f"act_{dt}_{n}"], z[f"y_{dt}_{n}"]
            got = oracle.matvec_rows(dt, W, W.shape[1], act, n, 0, W.shape[0])
            assert np.all(same(got, y)), (dt, n)


def golden_moe_host(z):
    E = z["gate"].shape[0]
    experts = [(z["gate"][e], z["up"][e], z["down"][e]) for e in range(E)]
    return oracle.MoeHost(D=256, de=256, E=E, k=2, expert_dt=Q6_K, ffn_norm=z["ffn_norm"], router_w=z["router_w"],
                          experts=experts, ds=256, shared_dt=Q8_0, shared=(z["sg"], z["su"], z["sd"]))


def test_oracle_moe_matches_golden():
    z = load("moe.npz")
    host = golden_moe_host(z)
    for t in range(z["h_in"].shape[0]):
        h, ids, w, _ = host.run(z["h_in"][t])
        assert np.array_equal(ids, z["ids"][t]) and np.array_equal(w, z["w"][t])
        assert np.array_equal(h.view(np.uint32), z["h_out"][t].view(np.uint32)), t


@pytest.mark.gpu
def test_hip_matches_golden(hip, dev):
    import torch
    z = load("dots.npz")
    for dt in INT:
        for n in (256, 768, 2048):
            W, act, y = z[f"w_{dt}_{n}"], z[f"act_{dt}_{n}"], z[f"y_{dt}_{n}"]
            Wd = torch.from_numpy(W.reshape(-1).copy()).to(dev)
            ad = torch.from_numpy(act.copy()).to(dev)
            plain = hip.matvec_rows(dt, Wd, W.shape[1], ad, n, 0, W.shape[0])
            packed = hip.matvec_packed(dt, hip.pack(dt, Wd, W.shape[1], W.shape[0], n), W.shape[0], n, ad)
            torch.cuda.synchronize()
            assert np.all(same(plain.cpu().numpy(), y)), (dt, n)
            assert np.all(same(packed.cpu().numpy()[:W.shape[0]], y)), (dt, n)
    z = load("act.npz")
    i = 0
    while f"x{i}" in z:
        x = torch.from_numpy(z[f"x{i}"].copy()).to(dev)
        for kind, key in ((Q8_K, "k"), (Q8_0, "a")):
            got = hip.quantize_act(kind, x)
            torch.cuda.synchronize()
            want = z[f"{key}{i}"]
            assert np.array_equal(got.cpu().numpy()[:want.size], want), (i, kind)
        i += 1


@pytest.mark.gpu
def test_hip_moe_matches_golden(hip, dev):
    import torch

    from tests.synth import device_block
    z = load("moe.npz")
    host = golden_moe_host(z)
    case = type("C", (), {})()
    case.D, case.de, case.ds, case.E, case.k = 256, 256, 256, z["gate"].shape[0], 2
    case.expert_dt, case.shared_dt = Q6_K, Q8_0
    case.experts = [(z["gate"][e], z["up"][e], z["down"][e]) for e in range(case.E)]
    case.shared = (z["sg"], z["su"], z["sd"])
    case.ffn_norm, case.router_w = z["ffn_norm"], z["router_w"]
    block, keep = device_block(case, dev)
    for t in range(z["h_in"].shape[0]):
        h = torch.from_numpy(z["h_in"][t].copy()).to(dev)
        block(h)
        torch.cuda.synchronize()
        got = h.cpu().numpy()
        want = z["h_out"][t]
        assert np.array_equal(block.ids.cpu().numpy()[:2], z["ids"][t])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (t, np.abs(got - want).max())
    _ = host
