"""The compiled C++ drop-in layer (include/ninfer_amd/ops.hpp) on the GPU: tests/cpp/ops_hpp_driver
runs A1 attention with a WorkspaceArena sized by the reference-signature query
gqa_attention_workspace_bytes(q_heads, tokens), argmax, greedy acceptance and the INT8 prefix commit,
exactly as a reference caller would; its outputs are compared here with the oracle (codes, scales,
tokens and stats bit-exact; attention within 2e-3 relative L2)."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from helpers import AttnCase, reference_composite_ok, rel_l2
from ninfer_amd import synthetic as syn

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent


def test_cpp_layer_runs_a_verify_step(gpu, oracle, tmp_path):
    exe = ROOT / "tests" / "cpp" / "ops_hpp_driver"
    assert exe.exists(), "build tests/cpp first (__graft_entry__.build())"
    L, T, K, V = 2500, 4, 3, 32768
    case = AttnCase([L], T=T, seed=808)
    P = case.P
    logits = syn.normal_bf16(81, V * (K + 1), 2.0)
    tgt = oracle.argmax(logits, V, K + 1, V)
    drafts = np.array([tgt[0], tgt[1], (tgt[2] + 1) % V], np.int32)  # two accepted, then a rejection
    k2 = syn.normal_bf16(82, 128 * 8 * T)
    v2 = syn.normal_bf16(83, 128 * 8 * T)
    pos2 = np.arange(L + T, L + 2 * T, dtype=np.int32)
    commit = 3
    for name, a in dict(q=case.q, k=case.k_new, v=case.v_new, positions=case.positions, kc=case.kc, vc=case.vc,
                        ks=case.ks, vs=case.vs, logits=logits, drafts=drafts, k2=k2, v2=v2, positions2=pos2).items():
        np.ascontiguousarray(a).tofile(tmp_path / f"{name}.bin")
    (tmp_path / "meta.txt").write_text(f"{L} {T} {case.max_context + T} {P} {V} {K} {L} {commit}\n")
    print("case cpp driver run", flush=True)
    r = subprocess.run([str(exe), "run", str(tmp_path)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and "RUN PASS" in r.stdout
    # attention and the A1 append
    (kc, vc, ks, vs), ref = case.oracle_after_append()
    out = np.fromfile(tmp_path / "out.bin", np.uint16)
    got = (out.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    assert rel_l2(got, ref) <= 2e-3
    ok, msg = reference_composite_ok(got, ref)
    assert ok, msg
    # acceptance
    assert list(np.fromfile(tmp_path / "target_out.bin", np.int32)) == list(tgt)
    exp = oracle.speculative_accept(tgt, logits, V, drafts, L, np.zeros(4 + K, np.int64), V, oracle.SamplingConfig())
    assert list(np.fromfile(tmp_path / "sampled_out.bin", np.int32)) == list(exp["sampled_out"])
    assert np.fromfile(tmp_path / "length_out.bin", np.int32)[0] == exp["length"]
    assert np.fromfile(tmp_path / "token_out.bin", np.int32)[0] == exp["token"]
    assert list(np.fromfile(tmp_path / "stats_out.bin", np.int64)) == list(exp["stats"])
    # prefix commit after the append
    oracle.kv_commit_prefix(k2, v2, pos2, T, commit, 8, 128, P, kc[0], vc[0], ks[0], vs[0])
    for name, want in (("kc", kc), ("vc", vc), ("ks", ks), ("vs", vs)):
        dt = np.int8 if name in ("kc", "vc") else np.uint16
        assert np.array_equal(np.fromfile(tmp_path / f"{name}_out.bin", dt), want.reshape(-1)), name
