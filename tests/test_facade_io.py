"""marisa::Trie::map / read / write (the reference's memory and descriptor
I/O, lib/marisa/trie.cc:33-43, 57-67, 78-86): a C++ program written as
reference code calls them, compiled against include/ and linked with
libmarisa_amd.so; and the same through the Python module.  No GPU."""

import os
import subprocess
import threading

import numpy as np

from helpers import assert_same_results

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "flash-trie_amd")


def test_reference_style_program(ft, tmp_path):
    exe = tmp_path / "facade_io"
    subprocess.check_call(
        ["g++", "-O1", "-std=c++17", "-I" + os.path.join(ROOT, "include"),
         os.path.join(ROOT, "tests", "native", "facade_io.cpp"), "-o", str(exe),
         "-L" + PKG, "-lmarisa_amd", "-lflashtrie_amd", "-Wl,-rpath," + PKG, "-lpthread"])
    p = subprocess.run([str(exe), str(tmp_path)], capture_output=True, text=True, timeout=60)
    assert p.returncode == 0 and "0 failures" in p.stdout, p.stdout + p.stderr


def _search(ft, t, ids, lp):
    return ft.tbs(t, [6] * ids.shape[0], ids, lp, -10.0, -40.0, 5.0, False, False)[:2]


def test_python_pipe_and_buffer(ft, tmp_path):
    toks, offs = ft.synth_keys(20000, 1024, 3, 8, 1.1, 3)
    a = ft.Trie()
    a.build_arrays(toks, offs)
    ids, lp = ft.synth_requests(a, 0, 3, 1024, 6, 24, 6, 0.3, 2.0, True, 1)
    want = [_search(ft, a, ids[r], lp[r]) for r in range(3)]
    marisa = a.marisa_bytes()
    # an image and a MARISA file back to back through one pipe
    r, w = os.pipe()

    def writer():
        a.write(w)
        os.write(w, marisa.tobytes())
        os.close(w)
    th = threading.Thread(target=writer)
    th.start()
    t1, t2 = ft.Trie(), ft.Trie()
    t1.read(r)
    t2.read(r)
    th.join()
    assert os.read(r, 1) == b""
    os.close(r)
    for t in (t1, t2):
        assert t.num_keys() == a.num_keys()
        for q in range(3):
            assert_same_results(_search(ft, t, ids[q], lp[q]), want[q])
    # a buffer in place: the image, and a MARISA file
    for buf in (a.image(), bytearray(marisa.tobytes())):
        m = ft.Trie()
        m.map(buf)
        del buf  # kept alive by the Trie
        for q in range(3):
            assert_same_results(_search(ft, m, ids[q], lp[q]), want[q])
