"""The benchmark's contract and accounting, on the CPU: one GPU only, the configurations it measures, and the
algorithmic bytes its roofline divides by (each declared input read once, each output written once)."""
import os
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 2 and "one GPU" in r.stderr


@pytest.mark.parametrize("cfg,shape", [
    (1, dict(B=4, T=1024, Hk=16, Hv=16, DK=128, DV=128, s0=False)),
    (2, dict(B=2, T=1024, Hk=16, Hv=32, DK=128, DV=128, s0=True)),
    (3, dict(B=1, T=32768, Hk=16, Hv=16, DK=128, DV=128, s0=False)),
    (4, dict(B=64, T=1, Hk=16, Hv=32, DK=128, DV=128, s0=True))])
def test_configs_are_the_baseline_shapes(cfg, shape):
    """BASELINE.json configs 1-4 (config 3 also runs at Hv = 32 through --hv)."""
    assert bench.CONFIGS[cfg] == shape


def test_training_step_bytes_per_chunk_head():
    """Config 1's training step as the library runs it (the forward keeping prep's operands and the chunk states):
    per chunk-head, prep with A 144.5 KiB, the state pass with the output and S_c, Vn 184.0 KiB, the reverse pass
    152.0 KiB, the chunk backward 281.0 KiB, from the tensors' sizes: q, k, v, dO 16 KiB a chunk-head each in bf16,
    g and beta 0.5 KiB, W, Ke, Qg 16 KiB, U 32 KiB (fp32), M and A 8 KiB, S_c and dS 64 KiB (fp32), Vn and dVn
    16 KiB, GL 4 bytes."""
    c = bench.CONFIGS[1]
    cost = bench.kernel_costs(c["B"], c["T"], c["Hv"], c["DK"], c["DV"], keep=True)
    n = c["B"] * c["Hv"] * (c["T"] // 64)
    kib = {k: cost[k]["bytes"] / n / 1024 for k in ("prep_fwd", "state_fwd_out", "state_bwd", "chunk_bwd")}
    assert kib["prep_fwd"] == pytest.approx(3 * 16 + 0.5 + 3 * 16 + 32 + 8 + 8 + 4 / 1024)
    assert kib["state_fwd_out"] == pytest.approx(3 * 16 + 32 + 8 + 4 / 1024 + 64 + 16 + 16)
    assert kib["state_bwd"] == pytest.approx(3 * 16 + 8 + 4 / 1024 + 64 + 16 + 16)
    assert kib["chunk_bwd"] == pytest.approx(3 * 16 + 0.5 + 16 + 8 + 2 * 64 + 2 * 16 + 3 * 16 + 0.5)
    assert [round(kib[k], 1) for k in kib] == [144.5, 184.0, 152.0, 281.0]


def test_decode_bytes():
    """Config 4: the fp32 state [64, 32, 128, 128] read and written (268.4 MB) plus the token tensors."""
    b = bench.decode_bytes(64, 32, 16, 128, 128)
    state = 64 * 32 * 128 * 128 * 4
    assert b == 2 * state + 64 * (2 * 16 * 128 + 2 * 32 * 128) * 2 + 64 * 32 * 8
    assert round(2 * state / 1e6, 1) == 268.4


def test_recompute_step_bytes_per_chunk_head():
    """Config 1 as BASELINE specifies it (the backward recomputes): prep without A 136.5 KiB, the output-only state
    pass 104.0 KiB, prep with A 144.5 KiB, the pair pass 296.0 KiB (recompute: W, Ke 16 KiB each, U 32 KiB, GL in;
    S_c 64 KiB and Vn 16 KiB out; and the reverse pass's 152.0 KiB), the chunk backward 281.0 KiB; reads and writes
    add up to the total."""
    c = bench.CONFIGS[1]
    cost = bench.kernel_costs(c["B"], c["T"], c["Hv"], c["DK"], c["DV"], keep=False)
    n = c["B"] * c["Hv"] * (c["T"] // 64)
    kib = {k: round(cost[k]["bytes"] / n / 1024, 1) for k in bench.step_kernels(False)}
    assert kib == {"prep_fwd": 136.5, "state_fwd_out": 104.0, "prep_bwd": 144.5, "state_pair": 296.0,
                   "chunk_bwd": 281.0}
    for keep in (False, True):
        for name, x in bench.kernel_costs(2, 100, 3, 128, 64, keep=keep, Hk=1).items():
            assert x["reads"] + x["writes"] == x["bytes"], name


def test_traffic_only_while_the_kernels_match(monkeypatch):
    """Counter traffic is reported only for the kernel sources it was profiled on."""
    fp = bench.kernel_fingerprint()
    monkeypatch.setattr(bench, "TRAFFIC", {(1, "recompute"): {"sources": fp, "bytes": {"chunk_bwd": 1.0}}})
    assert bench.measured_traffic(1, "recompute")["chunk_bwd"] == 1.0
    assert "chunk_bwd" not in bench.measured_traffic(1, "stored")
    monkeypatch.setattr(bench, "TRAFFIC", {(1, "recompute"): {"sources": "0" * 16, "bytes": {"chunk_bwd": 1.0}}})
    t = bench.measured_traffic(1, "recompute")
    assert "chunk_bwd" not in t and t["_source"].startswith("stale")


def test_cpu_info():
    model, physical, allowed, share = bench.cpu_info()
    assert physical >= 1 and allowed >= 1 and share >= 1 and isinstance(model, str)


def test_traffic_fingerprint_reads_code_not_comments():
    """The fingerprint hashes the kernel sources' code: comments, blank lines and indentation do not move it, a change
    of code does."""
    code = "int a = 1;  // one\n\n/* a block\n   comment */  int b = a;\n"
    assert bench.kernel_code(code) == "int a = 1;\nint b = a;"
    assert bench.kernel_code(code.replace("// one", "// uno")) == bench.kernel_code(code)
    assert bench.kernel_code(code.replace("a = 1", "a = 2")) != bench.kernel_code(code)


def test_traffic_fingerprint_covers_the_build_flags():
    """The traffic stamp's fingerprint includes build.py, whose compile flags (chunk_bwd8's scheduler strategy) change
    the generated code and so its traffic."""
    assert "build.py" in bench.KERNEL_SOURCES and len(bench.kernel_fingerprint()) == 16


def test_bench_draws_the_oracle_generators_inputs():
    """The bench's seeded CPU draw is the oracle's generator (same order, same seed, same values), so the driver's
    bench runs on the inputs the parity tests check."""
    from oracle import gdr
    mine, _ = bench.make_inputs(1, 1001, "cpu")
    ref = gdr.config_inputs(1)
    for n in ("query", "key", "value", "g", "beta", "do"):
        assert torch.equal(mine[n], ref[n]), n
