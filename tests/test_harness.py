"""The benchmark harness (flash-trie_amd/ft_harness.py, run_trie_search.py,
make_example_data.py, sweep.py): the same proposal files, request
preparation and latency files as the reference's examples/."""

import json
import math
import os
import subprocess
import sys

import numpy as np
import pytest

PKG = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                   "flash-trie_amd")
if PKG not in sys.path:
    sys.path.insert(0, PKG)

import ft_harness as H  # noqa: E402


def test_prepare_sorts_and_selects_superset():
    rec = {"indices": [[9, 3, 7, 1, 5], [2, 4, 6, 8, 10]],
           "probs": [[-1.0, -5.0, -0.5, -3.0, -2.0], [-9, -8, -7, -6, -5]]}
    beams, ids, lp, forced = H.prepare_request(rec, 4, 5)
    assert beams == [4, 4] and not forced
    assert ids[0] == [1, 3, 5, 7, 9]
    assert lp[0] == [-3.0, -5.0, -2.0, -0.5, -1.0]
    # the 3 best columns of each row, then token order
    _, ids, lp, _ = H.prepare_request(rec, 4, 3, superset_topk=True)
    assert ids == [[5, 7, 9], [6, 8, 10]]
    assert lp == [[-2.0, -0.5, -1.0], [-7.0, -6.0, -5.0]]
    with pytest.raises(ValueError, match="K=5"):
        H.prepare_request(rec, 4, 3)


@pytest.mark.parametrize("start", ["lcid", 2])
def test_prepare_forced_first_step(start):
    rec = {"indices": [[9, 3, 7]], "probs": [[-1.0, -2.0, -3.0]], "lcid": 2}
    beams, ids, lp, forced = H.prepare_request(rec, 8, 3, start_token=start)
    assert forced and beams == [1, 8]
    assert ids[0] == sorted(ids[0]) and 2 in ids[0] and len(set(ids[0])) == 3
    assert [x for t, x in zip(ids[0], lp[0]) if t == 2] == [0.0]
    assert all(math.isinf(x) and x < 0 for t, x in zip(ids[0], lp[0]) if t != 2)
    assert ids[1] == [3, 7, 9]


def test_read_topk_tsv_and_batches(tmp_path):
    p = tmp_path / "t.tsv"
    p.write_text('q0\t{"probs": [[-1]], "indices": [[4]]}\n\nq1\t{"probs": [[-2]], '
                 '"indices": [[5]]}\nq2\t{"probs": [[-3]], "indices": [[6]]}\n')
    rows = list(H.read_topk_tsv(str(p)))
    assert [q for q, _ in rows] == ["q0", "q1", "q2"]
    assert rows[1][1]["indices"] == [[5]]
    assert len(list(H.read_topk_tsv(str(p), max_queries=2))) == 1  # line 2 is blank
    assert [len(b) for b in H.iter_batches(range(7), 3)] == [3, 3, 1]
    p.write_text("no tab here\n")
    with pytest.raises(ValueError, match="TAB"):
        list(H.read_topk_tsv(str(p)))


def test_summarize_latency_by_hand():
    runs = [[1.0, 2.0, 3.0, 4.0], [2.0, 2.0, 2.0, 6.0]]
    s = H.summarize_latency(runs, (50,))
    assert s["num_measured_runs"] == 2
    assert s["mean_ms"] == pytest.approx(2.75)             # means 2.5 and 3.0
    assert s["std_ms"] == pytest.approx(math.sqrt(0.125))  # sample std of the two
    assert s["p50_ms"] == pytest.approx(2.25)              # medians 2.5 and 2.0
    head, row = H.latency_tsv(10, 8, 1, 4, H.summarize_latency(runs), 100.0, 1.5)
    cols = head.split("\t")
    assert cols[:7] == ["beam", "topk", "batch_size", "batches_per_run",
                        "num_measured_runs", "mean_ms", "std_ms"]
    assert cols[-2:] == ["mean_qps", "std_qps"] and len(cols) == 17
    assert row.split("\t")[:6] == ["10", "8", "1", "4", "2", "2.750"]


def _run(script, *args):
    p = subprocess.run([sys.executable, os.path.join(PKG, script), *args],
                       capture_output=True, text=True, timeout=600)
    assert p.returncode == 0, p.stdout[-3000:] + p.stderr[-3000:]
    return p.stdout


@pytest.fixture(scope="module")
def example(tmp_path_factory, ft):
    d = tmp_path_factory.mktemp("example")
    _run("make_example_data.py", "--out-dir", str(d), "--num-keys", "30000",
         "--num-queries", "16", "--topk", "48", "--seeds-per-query", "24",
         "--write-keys", "--vocab-size", "50000")
    return d


def test_example_data_files(ft, example):
    t = ft.Trie()
    t.load(str(example / "trie.bin"))
    with open(example / "trie.bin", "rb") as f:
        assert f.read(16) == b"We love Marisa.\0"
    keys = [list(map(int, ln.split())) for ln in open(example / "keys.txt")]
    assert len(keys) == 30000 == t.num_keys()
    rows = list(H.read_topk_tsv(str(example / "topk.tsv")))
    assert [q for q, _ in rows] == [f"query_{i}" for i in range(16)]
    r = rows[0][1]
    assert np.asarray(r["indices"]).shape == (8, 48)
    for ids in r["indices"]:
        assert ids == sorted(ids) and len(set(ids)) == 48


def test_run_cpu_end_to_end(ft, example, tmp_path):
    out, lat = tmp_path / "out.tsv", tmp_path / "lat.tsv"
    _run("run_trie_search.py", "--trie-path", str(example / "trie.bin"), "--data-path",
         str(example / "topk.tsv"), "--beam-size", "16", "--topk-tokens", "32",
         "--superset-topk", "--cpu", "--num-runs", "2", "--batch-size", "4",
         "--output-path", str(out), "--latency-out", str(lat))
    lines = out.read_text().splitlines()
    assert len(lines) == 16
    # every line = the host search of that prepared request
    t = ft.Trie()
    t.load(str(example / "trie.bin"))
    rows = list(H.read_topk_tsv(str(example / "topk.tsv")))
    for (q, rec), ln in zip(rows, lines):
        beams, ids, lp, _ = H.prepare_request(rec, 16, 32, superset_topk=True)
        sents, _, _ = ft.tbs(t, beams, ids, lp, -10.0, -40.0, 5.0, False)
        seqs = " | ".join(" ".join(map(str, s)) for s in sents)
        assert ln == f"{q}\t{len(sents)}\t{seqs}"
    head, row = lat.read_text().splitlines()
    assert head.split("\t")[0] == "beam" and row.split("\t")[:4] == ["16", "32", "4", "4"]


def test_forced_prefix_strips_the_token(ft, tmp_path):
    # keys behind a prefix token 77: a forced first step reaches them and the
    # results come back without the 77
    keys = [[1, 2], [1, 3], [4]]
    t = ft.Trie()
    t.build([[77] + k for k in keys])
    p = tmp_path / "trie.img"
    t.save(str(p))
    s = H.Searcher(str(p), beam_size=4, topk_tokens=3, use_gpu=False,
                   trie_start_token="lcid", verbose=False)
    rec = {"lcid": 77, "indices": [[1, 4, 9], [2, 3, 9]],
           "probs": [[-0.5, -1.0, -2.0], [-0.1, -0.2, -3.0]]}
    seqs, scores = s.search([rec])
    assert sorted(seqs[0]) == [[1, 2], [1, 3], [4]]


def test_sweep_cpu(ft, example, tmp_path):
    d = tmp_path / "sweep"
    rep = tmp_path / "report.tsv"
    _run("sweep.py", "--trie-path", str(example / "trie.bin"), "--data-path",
         str(example / "topk.tsv"), "--beam-topk", "8:16", "16:32", "--superset-topk",
         "--batch-sizes", "1,4", "--cpu", "--num-runs", "2", "--output-dir", str(d),
         "--latency-report", str(rep))
    rows = rep.read_text().splitlines()
    assert len(rows) == 5
    assert sorted(os.listdir(d)) == sorted(f"latency_b{b}_k{k}_bs{bs}.tsv"
                                           for b, k in ((8, 16), (16, 32)) for bs in (1, 4))


@pytest.mark.gpu
def test_run_gpu_matches_cpu(ft, example, tmp_path):
    # the harness's functions in this process (the command line tool has
    # its own test)
    import run_trie_search
    outs = {}
    for dev in ("gpu", "cpu"):
        o = tmp_path / f"{dev}.tsv"
        args = ["--trie-path", str(example / "trie.bin"), "--data-path",
                str(example / "topk.tsv"), "--beam-size", "16", "--topk-tokens", "32",
                "--superset-topk", "--num-runs", "2", "--batch-size", "4",
                "--output-path", str(o), "--phase-out", str(tmp_path / f"{dev}_ph.tsv")]
        assert run_trie_search.main(args + (["--cpu"] if dev == "cpu" else [])) == 0
        outs[dev] = o.read_text()
    assert outs["gpu"] == outs["cpu"]
    head, row = (tmp_path / "gpu_ph.tsv").read_text().splitlines()
    assert head.split("\t")[3:] == [f"{n}_ms" for n in H.PHASE_NAMES]
