"""The cross-workgroup protocol of the search kernel (claims, done words,
the shared step's parameters and pushes) relies on how the compiler lowers
coherent.h's primitives for gfx950: a relaxed agent-scope load or store
becomes one global load / store with the `sc1` bit (served at the agent's
coherence point, not from a stale line of another XCD's L2), with no cache
write-back or invalidate around it, and the store wait is a bare
`s_waitcnt vmcnt(0)` that stays between the data stores and the signal.
This compiles probe kernels made of those primitives alone (CPU only:
hipcc cross-compiles) and checks the instructions, so that a compiler that
lowered them otherwise fails here instead of silently."""

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _functions(asm):
    """Kernel name -> its instruction lines, from a gfx950 assembly listing."""
    out, name = {}, None
    for line in asm.splitlines():
        m = re.match(r"^(_Z\w+):", line)
        if m:
            name = m.group(1)
            out[name] = []
        elif name and line.startswith("\t") and not line.lstrip().startswith((".", ";")):
            out[name].append(line.strip())
        if name and line.startswith(".Lfunc_end"):
            name = None
    return out


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not (os.path.exists(HIPCC) or shutil.which("hipcc")):
        pytest.skip("no hipcc")
    d = tmp_path_factory.mktemp("probe")
    out = d / "probe.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "--offload-device-only",
           "-S", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I" + os.path.join(ROOT, "flash-trie_amd", "csrc"), "-o", str(out),
           os.path.join(ROOT, "tests", "native", "coherence_probe.hip")]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return _functions(out.read_text())


def _one(fn, pattern):
    hits = [i for i in fn if re.search(pattern, i)]
    assert len(hits) == 1, (pattern, fn)
    return hits[0]


def _no_cache_maintenance(fn):
    assert not [i for i in fn if i.startswith(("buffer_wbl2", "buffer_inv", "buffer_wbinv"))], fn


@pytest.mark.parametrize("kernel,op", [("probe_ld32", r"^global_load_dword\s"),
                                       ("probe_ld64", r"^global_load_dwordx2\s")])
def test_relaxed_loads_are_sc1_loads(asm, kernel, op):
    fn = next(v for k, v in asm.items() if kernel in k)
    assert re.search(r"\bsc1\b", _one(fn, op))
    _no_cache_maintenance(fn)


@pytest.mark.parametrize("kernel,op", [("probe_st32", r"^global_store_dword\s"),
                                       ("probe_st64", r"^global_store_dwordx2\s")])
def test_relaxed_stores_are_sc1_stores(asm, kernel, op):
    fn = next(v for k, v in asm.items() if kernel in k)
    assert re.search(r"\bsc1\b", _one(fn, op))
    _no_cache_maintenance(fn)


def test_signal_follows_the_store_wait(asm):
    fn = next(v for k, v in asm.items() if "probe_signal" in k)
    stores = [n for n, i in enumerate(fn) if i.startswith("global_store_dword")]
    assert len(stores) == 2 and all(re.search(r"\bsc1\b", fn[n]) for n in stores), fn
    wait = [n for n, i in enumerate(fn) if i == "s_waitcnt vmcnt(0)"]
    barrier = [n for n, i in enumerate(fn) if i == "s_barrier"]
    # data store < vmcnt(0) wait < barrier < flag store
    assert wait and barrier, fn
    assert stores[0] < wait[0] < barrier[0] < stores[1], fn
    _no_cache_maintenance(fn)
