"""Host logic of the evaluation harness (amd_optimization_challenge_amd/harness.py):
spec parsing, seed mixing, Stats, the match rules, and the torch checker
pinned against the oracle on the CPU (no device calls)."""
import math

import numpy as np
import pytest
import torch

from amd_optimization_challenge_amd import harness as Hn
from oracle import mla_oracle as O


def test_parse_specs_types_and_errors():
    cases = Hn.parse_specs("batchsize: 4; qseqlen: 1; kvseqlen: 1024; seed: -7\n\nflag: true; name: fp8\n")
    assert [c.args for c in cases] == [dict(batchsize=4, qseqlen=1, kvseqlen=1024, seed=-7),
                                       dict(flag=True, name="fp8")]
    assert cases[0].spec.startswith("batchsize: 4")
    for bad in ("batchsize 4", "4x: 1", "a: 1.5", "a: b c", "a: 1;"):
        with pytest.raises(ValueError):
            Hn.parse_specs(bad)
    # the built-in lists round-trip through the spec format
    for kind in ("test", "benchmark"):
        cases = Hn.task_cases(kind)
        assert [c.args for c in Hn.parse_specs("\n".join(c.spec for c in cases))] == [c.args for c in cases]
    assert len(Hn.task_cases("benchmark")) == 8 and len(Hn.task_cases("test")) == 4


def test_seed_mix_is_an_injective_pairing():
    seen = {Hn.mix_seed(a, b) for a in range(60) for b in range(60)}
    assert len(seen) == 3600
    assert Hn.mix_seed(0, 0) == 0 and Hn.mix_seed(1, 0) == 2 and Hn.mix_seed(0, 1) == 1
    c = Hn.task_cases("test", secret=1234)
    assert c[0].args["seed"] == Hn.mix_seed(Hn.TASK_TESTS[0]["seed"], 1234) != Hn.TASK_TESTS[0]["seed"]


def test_stats_match_numpy():
    d = [5.0, 7.0, 6.5, 9.25, 4.0]
    st = Hn.calculate_stats(d)
    assert st.runs == 5 and st.mean == pytest.approx(np.mean(d))
    assert st.std == pytest.approx(np.std(d, ddof=1)) and st.err == pytest.approx(np.std(d, ddof=1) / math.sqrt(5))
    assert (st.best, st.worst) == (4.0, 9.25)
    assert Hn.calculate_stats([3.0]).std == 0.0
    assert Hn.geomean([1.0, 100.0]) == pytest.approx(10.0)


def test_match_rules():
    exp = torch.ones(1000, dtype=torch.bfloat16)
    good, msg = Hn.match(exp.clone(), exp)
    assert good and msg.startswith("Maximum error")
    out = exp.clone()
    out[:40] = 2.0                                      # 4 % off: passes with a warning
    good, msg = Hn.match(out, exp)
    assert good and "mismatch_ratio=0.040000" in msg
    out[:60] = 2.0                                      # 6 % off: fails
    good, msg = Hn.match(out, exp)
    assert not good and "Number of mismatched elements: 60" in msg
    nan = exp.clone()
    nan[3] = float("nan")
    assert Hn.match(nan, exp)[0]                        # one NaN is within the 5 % allowance
    assert not Hn.match(torch.ones(10), torch.ones(11))[0]
    out = exp.clone() * 1.09                            # inside rtol = atol = 0.1
    assert Hn.match(out, exp)[0]


def _cpu_case(lens, qlen, seed, permute):
    g = torch.Generator().manual_seed(seed)
    S, H = len(lens), 16
    T = sum(lens)
    q = torch.randn((S * qlen, H, 576), generator=g, dtype=torch.bfloat16)
    kv = torch.randn((T, 1, 576), generator=g, dtype=torch.bfloat16)
    idx = torch.randperm(T, generator=g).to(torch.int32) if permute else None
    codes, s = O.quantize_fp8_per_tensor(O.bf16_tensor_bits(kv).reshape(T, 576))
    fp8 = torch.from_numpy(codes.reshape(T, 1, 576)).view(torch.float8_e4m3fn)
    indptr = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    cfg = {"q_seq_len": qlen, "sm_scale": 1 / math.sqrt(576), "kv_indices": idx}
    data = (q, {"fp8": (fp8, torch.tensor([s], dtype=torch.float32))}, None, indptr, cfg)
    return data, codes, s


@pytest.mark.parametrize("lens,qlen,permute", [([40, 40, 40], 1, False), ([33, 1, 70], 1, True),
                                               ([16, 16], 2, False), ([5, 1, 9], 4, True)])
def test_torch_checker_matches_oracle(lens, qlen, permute):
    """The checker's a8w8 arithmetic against the oracle's reference path (same
    fp8 Q and KV by construction, both f32); outputs agree to bf16 rounding."""
    data, codes, s = _cpu_case(lens, qlen, 3 + len(lens), permute)
    q, _, _, indptr, cfg = data
    got = Hn.reference_kernel(data).float().numpy()
    idx = np.arange(sum(lens), dtype=np.int32) if cfg["kv_indices"] is None else cfg["kv_indices"].numpy()
    _, ref = O.reference_path(O.bf16_tensor_bits(q), "fp8", {"fp8_codes": codes, "fp8_scale": s},
                              indptr.numpy(), idx, cfg["sm_scale"], q_seq_len=qlen)
    ref_b = O.bf16_to_f32(O.f32_to_bf16(ref))
    assert np.abs(got - ref_b).max() <= 2 ** -7 * np.abs(ref_b).max() + 1e-6
    if qlen > 1:  # rows whose causal prefix is empty are zero in both
        assert np.array_equal(got == 0, ref_b == 0)


def test_torch_quantizer_is_the_reference_expression():
    """The checker's Q quantizer gives the oracle's bytes and scale."""
    g = torch.Generator().manual_seed(9)
    x = torch.randn((7, 16, 576), generator=g, dtype=torch.bfloat16) * 3
    q8, sc = Hn._quantize_fp8_torch(x)
    codes, s = O.quantize_fp8_per_tensor(O.bf16_tensor_bits(x))
    assert np.array_equal(q8.view(torch.uint8).numpy().reshape(-1), codes.reshape(-1))
    assert float(sc) == float(s)
