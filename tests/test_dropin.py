"""The drop-in: the reference's own `tierlm` with libtlm_hip.so taken into its
kernel dispatch and its decode step (oracle/dropin.py builds it from a
build-directory copy of the reference's sources), run on the 4-layer
synthetic store (oracle/make_c1.sh) against the reference's own outputs
(tests/golden/make_c1_golden.sh):

* --kernel hip: tlm_quant_tier() is "hip" with no self-test failures (the
  reference's bit-exact self-test, src/lib/tlm_quant.c:1015-1056, run over
  the HIP entries), and tlm_model_step runs the whole step on the device:
  `tierlm run` gives the reference's 64 greedy tokens, `tierlm oracle` its
  teacher-forced top-10 logits text for text (9 significant digits, so bit
  for bit), `tierlm bench` runs its loop;
* on C2S (oracle/make_c2s.sh), whose geometry the batched prefill takes,
  tlm_model_prefill hands the prompt to tlm_hip_model_prefill: `tierlm run`
  gives the reference's greedy tokens;
* TIERLM_HIP_TIER_ONLY=1 --kernel hip: the reference's own CPU step with
  every quantised matvec of its kernel table on the device (the host-pointer
  entries of tlm_kern_hip_fill): the same tokens;
* --cache below the experts' size: the runtime's budget (raised to top_k
  slots) becomes the device's HBM slot cache - on C1 and on C3S (Qwen3-30B-
  A3B's attention geometry) `tierlm run` gives the reference's greedy tokens
  and `tierlm oracle` its top-10 text, and --stats reports the device
  cache's hits, misses and evictions and the device step's attention / MoE
  split;
* on C6D (oracle/make_c6d.sh), two dense-FFN layers before the MoE layers:
  `tierlm oracle` gives the reference's top-10 text with every expert
  resident, and `tierlm run` its greedy tokens through 4 slots."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TIERLM = os.path.join(ROOT, "oracle", "_ref", "dropin", "bin", "tierlm")
C1 = os.path.join(ROOT, "oracle", "_ref", "c1", "c1.tlmm")
GOLD = os.path.join(ROOT, "tests", "golden")
C2S = os.path.join(ROOT, "oracle", "_ref", "c2s", "c2s.tlmm")
C6D = os.path.join(ROOT, "oracle", "_ref", "c6d", "c6d.tlmm")
needs = pytest.mark.skipif(not (os.path.exists(TIERLM) and os.path.exists(C1)),
                           reason="oracle/_ref/dropin (python3 oracle/dropin.py) or oracle/_ref/c1 not built")


def prompt_ids(n=64, vocab=4096):
    x, out, m = 42, [], (1 << 64) - 1
    for _ in range(n):   # src/bin/tierlm.c:711-715
        x ^= (x << 13) & m
        x ^= x >> 7
        x ^= (x << 17) & m
        out.append(x % vocab)
    return out


def golden(name):
    return open(os.path.join(GOLD, name)).read()


def tierlm(args, env=None):
    e = dict(os.environ)
    e.update(env or {})
    r = subprocess.run([TIERLM] + args, capture_output=True, text=True, timeout=300, env=e)
    assert r.returncode == 0, f"tierlm {' '.join(args[:2])} failed ({r.returncode}): {r.stderr[-2000:]}"
    return r


@needs
def test_run_hip_step_greedy_tokens():
    p = ",".join(map(str, prompt_ids()))
    r = tierlm(["run", C1, "--tokens", p, "-n", "64", "--print-tokens", "--cache", "1G", "--kernel", "hip",
                "--stats"])
    assert r.stdout.split() == golden("c1_greedy.txt").split()
    assert "kernel hip (self-test failures 0)" in r.stderr, r.stderr[-1500:]


@needs
def test_oracle_hip_step_top10_text_identical():
    gen = golden("c1_greedy.txt").split()[:63]
    toks = ",".join(map(str, prompt_ids())) + "," + ",".join(gen)
    r = tierlm(["oracle", C1, "--tokens", toks, "--cache", "1G", "--kernel", "hip"])
    want = golden("c1_oracle.jsonl").splitlines()
    got = r.stdout.splitlines()
    assert len(got) == len(want) == 127
    bad = [i for i, (a, b) in enumerate(zip(got, want)) if a != b]
    assert not bad, f"{len(bad)} positions differ, first {bad[0]}: {got[bad[0]]} vs {want[bad[0]]}"


@needs
def test_run_hip_tier_only_greedy_tokens():
    p = ",".join(map(str, prompt_ids()))
    r = tierlm(["run", C1, "--tokens", p, "-n", "64", "--print-tokens", "--cache", "1G", "--kernel", "hip",
                "--stats"], env={"TIERLM_HIP_TIER_ONLY": "1"})
    assert r.stdout.split() == golden("c1_greedy.txt").split()
    assert "kernel hip (self-test failures 0)" in r.stderr, r.stderr[-1500:]


@needs
def test_bench_hip_step():
    r = tierlm(["bench", C1, "--prompt-len", "64", "-n", "64", "--cache", "1G", "--kernel", "hip"])
    line = r.stdout.splitlines()[0]
    assert "decode 64 tokens in" in line, r.stdout
    assert "kernel hip (self-test failures 0)" in r.stdout, r.stdout[-1500:]
    dec = float(line.split("decode 64 tokens in")[1].split("(")[1].split(" tok/s")[0])
    print(f"tierlm bench --kernel hip: {line}")
    assert dec > 0


@pytest.mark.skipif(not (os.path.exists(TIERLM) and os.path.exists(C2S)), reason="oracle/_ref/dropin or c2s not built")
def test_run_hip_batched_prefill_c2s():
    p = ",".join(map(str, prompt_ids(64, 2048)))
    r = tierlm(["run", C2S, "--tokens", p, "-n", "64", "--print-tokens", "--cache", "1G", "--kernel", "hip"])
    assert r.stdout.split() == golden("c2s_greedy.txt").split()


C3S = os.path.join(ROOT, "oracle", "_ref", "c3s", "c3s.tlmm")


def stats_fields(text):
    """the store / cache / per-token lines of tierlm --stats"""
    out = {}
    for line in text.splitlines():
        if line.startswith("store "):
            parts = line.split()
            out["hits"] = int(parts[2].rstrip(","))
            out["misses"] = int(parts[4])
            out["evictions"] = int(line.split("evictions ")[1].split(",")[0])
        elif line.startswith("cache "):
            out["slots"] = int(line.split()[1])
        elif line.startswith("per token"):
            out["attn_ms"] = float(line.split("attention ")[1].split(" ms")[0])
            out["moe_ms"] = float(line.split("moe ")[1].split(" ms")[0])
    return out


@needs
def test_run_hip_slot_cache_c1():
    """--cache 1 (raised to top_k = 4 slots of the 128 experts): the
    reference's greedy tokens and top-10 text through the device's slot
    cache, whose counters the stats print."""
    p = ",".join(map(str, prompt_ids()))
    r = tierlm(["run", C1, "--tokens", p, "-n", "64", "--print-tokens", "--cache", "1", "--kernel", "hip",
                "--stats"])
    assert r.stdout.split() == golden("c1_greedy.txt").split()
    st = stats_fields(r.stderr)
    assert st["slots"] == 4, r.stderr[-1500:]
    assert st["misses"] > 0 and st["evictions"] > 0, r.stderr[-1500:]
    assert st["attn_ms"] > 0 and st["moe_ms"] > 0, r.stderr[-1500:]
    gen = golden("c1_greedy.txt").split()[:63]
    toks = ",".join(map(str, prompt_ids())) + "," + ",".join(gen)
    r = tierlm(["oracle", C1, "--tokens", toks, "--cache", "1", "--kernel", "hip"])
    assert r.stdout.splitlines() == golden("c1_oracle.jsonl").splitlines()


@pytest.mark.skipif(not (os.path.exists(TIERLM) and os.path.exists(C3S)), reason="oracle/_ref/dropin or c3s not built")
def test_run_hip_slot_cache_c3s():
    """Qwen3-30B-A3B's attention geometry with 16 experts top-8 through 8
    slots: the reference's 128 greedy tokens after the 1920-token prompt."""
    p = ",".join(map(str, prompt_ids(1920, 2048)))
    r = tierlm(["run", C3S, "--tokens", p, "-n", "128", "--print-tokens", "--cache", "1", "--kernel", "hip",
                "--stats"])
    assert r.stdout.split() == golden("c3s_greedy.txt").split()
    st = stats_fields(r.stderr)
    assert st["slots"] == 8 and st["misses"] > 0 and st["evictions"] > 0, r.stderr[-1500:]


@pytest.mark.skipif(not (os.path.exists(TIERLM) and os.path.exists(C6D)), reason="oracle/_ref/dropin or c6d not built")
def test_dense_ffn_layers_c6d():
    """Two dense-FFN layers before the MoE layers: the reference's
    teacher-forced top-10 text line for line with every expert in HBM, and
    its 64 greedy tokens after the 200-token prompt through 4 slots."""
    gen = golden("c6d_greedy.txt").split()
    p = ",".join(map(str, prompt_ids(200, 2048)))
    r = tierlm(["oracle", C6D, "--tokens", p + "," + ",".join(gen[:63]), "--cache", "1G", "--kernel", "hip"])
    want = golden("c6d_oracle.jsonl").splitlines()
    got = r.stdout.splitlines()
    assert len(got) == len(want) == 263
    bad = [i for i, (a, b) in enumerate(zip(got, want)) if a != b]
    assert not bad, f"{len(bad)} positions differ, first {bad[0]}: {got[bad[0]]} vs {want[bad[0]]}"
    r = tierlm(["run", C6D, "--tokens", p, "-n", "64", "--print-tokens", "--cache", "1", "--kernel", "hip",
                "--stats"])
    assert r.stdout.split() == gen
    st = stats_fields(r.stderr)
    assert st["slots"] == 4 and st["misses"] > 0, r.stderr[-1500:]
