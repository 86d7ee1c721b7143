"""The beam-search command line tool (ft-beam-search, the reference's
tools/marisa-beam-search.cc) and the proposal-file loader it shares with the
Python module (tools/beam-search-helper.h:26-120)."""

import os
import subprocess

import numpy as np
import pytest

PKG = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                   "flash-trie_amd")
CLI = os.path.join(PKG, "ft-beam-search")


def write_dataset(ft, d, n_req=12, T=6, K=24, seed=0):
    """marisa_trie.bin + topk_keys.txt / topk_scores.txt; rows after depth 0
    written in descending score order, as the loader expects."""
    toks, offs = ft.synth_keys(20000, 2048, 2, T, 1.1, seed)
    t = ft.Trie()
    t.build_arrays(toks, offs)
    t.save_marisa(os.path.join(d, "marisa_trie.bin"))
    ids, lp = ft.synth_requests(t, 0, n_req, 2048, T, K, 8, 0.3, 2.0, True, 3, model=1)
    with open(os.path.join(d, "topk_keys.txt"), "w") as kf, \
            open(os.path.join(d, "topk_scores.txt"), "w") as sf:
        kf.write(f"{n_req} {T} {K}\n")
        sf.write(f"{n_req} {T} {K}\n")
        for r in range(n_req):
            for s in range(T):
                o = np.argsort(-lp[r, s], kind="stable")
                kf.write(" ".join(str(int(x)) for x in ids[r, s, o]) + "\n")
                sf.write(" ".join(repr(float(x)) for x in lp[r, s, o]) + "\n")
    return t, ids, lp


def test_loader_sorts_rows_after_depth0(ft, tmp_path):
    t, ids, lp = write_dataset(ft, str(tmp_path))
    keys, scores = ft.load_topk_keys_and_scores(str(tmp_path))
    assert len(keys) == 12 and len(keys[0]) == 6 and len(keys[0][0]) == 24
    for r in range(12):
        # depth 0 keeps the file order (descending score); later rows are
        # sorted by token id, scores carried along
        o = np.argsort(-lp[r, 0], kind="stable")
        assert keys[r][0] == ids[r, 0, o].tolist()
        for s in range(1, 6):
            assert keys[r][s] == sorted(ids[r, s].tolist())
            m = dict(zip(ids[r, s].tolist(), lp[r, s].tolist()))
            assert scores[r][s] == [m[k] for k in keys[r][s]]


def test_loader_errors(ft, tmp_path):
    with pytest.raises(RuntimeError, match="cannot open"):
        ft.load_topk_keys_and_scores(str(tmp_path))
    (tmp_path / "topk_keys.txt").write_text("1 1 2\n3 4\n")
    (tmp_path / "topk_scores.txt").write_text("1 1 3\n-1 -2\n")
    with pytest.raises(RuntimeError, match="differ"):
        ft.load_topk_keys_and_scores(str(tmp_path))


def run_cli(*args):
    return subprocess.run([CLI, *args], capture_output=True, text=True, timeout=300)


def test_cli_host_search(ft, tmp_path):
    t, ids, lp = write_dataset(ft, str(tmp_path))
    p = run_cli(str(tmp_path), "8")
    assert p.returncode == 0, p.stderr
    lines = p.stdout.splitlines()
    assert lines[0] == f"Trie path {tmp_path}/marisa_trie.bin"
    reqs = [ln for ln in lines if ln.startswith("Req #")]
    assert len(reqs) == 12
    # the beam counts the tool prints are the host search's
    keys, scores = ft.load_topk_keys_and_scores(str(tmp_path))
    for r, ln in enumerate(reqs):
        sents, _, _ = ft.tbs(t, [8] * 6, keys[r], scores[r], -7.0, -40.0, 5.0, False)
        assert ln.startswith(f"Req #{r}: {len(sents)} beams generated in ")
    assert "Measured time per request in CPU tbs:" in lines[-1]


def test_cli_usage_errors(ft, tmp_path):
    assert run_cli().returncode == 10
    assert run_cli("a", "1", "2", "3").returncode == 11
    assert run_cli(str(tmp_path)).returncode == 21       # no marisa_trie.bin
    assert run_cli("-m", str(tmp_path)).returncode == 20
    assert run_cli("--bogus", str(tmp_path)).returncode == 1
    h = run_cli("-h")
    assert h.returncode == 0 and "--check-accuracy" in h.stderr


@pytest.mark.gpu
def test_cli_gpu_matches_host(ft, tmp_path):
    # The tool is a separate process searching on the GPU.
    write_dataset(ft, str(tmp_path))
    csv = tmp_path / "timing.csv"
    env = dict(os.environ, TBS_TIMING_CSV=str(csv))
    for early in ([], ["-e"]):
        p = subprocess.run([CLI, "-g", "-a", *early, str(tmp_path), "8", "4"],
                           capture_output=True, text=True, timeout=300, env=env)
        assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-2000:]
        assert "12/12 requests identical on CPU and GPU" in p.stdout
        rows = csv.read_text().splitlines()
        assert rows[0].startswith("req_id,beam_width,batch_size,num_beams,kernel_ms")
        assert len(rows) == 13
