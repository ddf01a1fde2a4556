"""bench.py's host-side contract, on the CPU: the one-GPU guard, the reference's
FLOP/byte conventions (bench/bench.py:153, 199-200) against the oracle's and
against the BASELINE configs' closed-form totals, the GPU accuracy reference
(a torch fp32 restatement) against the oracle, and the traffic table's entries."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import bench
import oracle
from conftest import ROOT

WORKLOADS = ["prefill_d128_n8192_causal", "prefill_d64_n2048", "prefill_d128_n8191_causal",
             "decode_ragged64_d128", "decode_long8_d128", "decode_long8_d64", "decode_gqa16_d128", "decode_g8_d128",
             "prefill_varlen_gqa", "cache_write_t16k"]


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}), ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused(args, env):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                       env={**os.environ, **env}, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_prefill_flop_convention():
    # causal B=2 H=32 N=8192 D=128 and non-causal B=4 H=16 N=2048 D=64.
    assert bench.prefill_flops(2, 32, 8192, 128, True) == pytest.approx(1.0995e12, rel=1e-4)
    assert bench.prefill_flops(4, 16, 2048, 64, False) == pytest.approx(6.872e10, rel=1e-4)
    for args in [(2, 32, 8191, 128, True), (1, 4, 256, 64, False), (3, 5, 17, 64, True)]:
        assert bench.prefill_flops(*args) == pytest.approx(oracle.prefill_flops(*args), rel=1e-12)


def test_decode_byte_convention():
    # 8 x 32768 tokens, 32 kv heads: 4.295 GB of K+V at D=128 and 2.147 GB at D=64.
    assert bench.decode_kv_bytes([32768] * 8, 32, 128) == 4294967296
    assert bench.decode_kv_bytes([32768] * 8, 32, 64) == 2147483648
    lens = list(np.random.default_rng(4).integers(1, 4097, 64))
    assert bench.decode_kv_bytes(lens, 32, 128) == oracle.decode_kv_bytes(lens, 32, 128)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n,d", [(1, 64), (77, 64), (130, 128)])
def test_accuracy_reference_matches_the_oracle(causal, n, d):
    g = torch.Generator().manual_seed(n + d)
    q, k, v = (torch.randn(n, d, generator=g).half() for _ in range(3))
    got = bench.torch_attention_fp32(q, k, v, causal, d ** -0.5).numpy()
    want = oracle.attention_fp32(q.numpy(), k.numpy(), v.numpy(), causal)
    assert np.abs(got - want).max() < 1e-5


def test_traffic_table_covers_every_workload():
    table = json.loads((ROOT / "profiles" / "traffic.json").read_text())
    for w in WORKLOADS:
        e = bench.measured_traffic(w)
        assert e is not None and e == table[w], w
        assert abs(e["traffic_bytes"] - (e["fetch_bytes"] + e["write_bytes"])) <= 1  # byte rounding
        assert (ROOT / e["source"]).exists(), e["source"]
