"""Build recipe for the MI355X trie beam search libraries (in-tree).

Outputs, next to this file:
  libflashtrie_amd.so   C ABI + HIP kernels (hipcc, gfx950)
  libmarisa_amd.so      drop-in marisa::Trie, image builder, generators (g++)
  flashtrie*.so         the `flashtrie` Python module (pybind11)
  ft_copy_calib         plain copy kernel of known size (HBM counter scale)

Run ``python flash-trie_amd/build.py`` or call ``build()``.
"""

import hashlib
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
INC = os.path.join(ROOT, "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = "gfx950"

# Device flags: no packed-FP32 instruction selection, no FMA contraction (the
# scores must round exactly like the reference's host arithmetic).
HIP_FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC",
             "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-I" + INC, "-I" + CSRC]
CXX_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-fopenmp", "-ffp-contract=off",
             "-Wall", "-Wno-unused-parameter", "-I" + INC, "-I" + CSRC]

LIB_AMD = os.path.join(HERE, "libflashtrie_amd.so")
LIB_MARISA = os.path.join(HERE, "libmarisa_amd.so")
COPY_CALIB = os.path.join(HERE, "ft_copy_calib")
BEAM_CLI = os.path.join(HERE, "ft-beam-search")


def ext_suffix():
    return sysconfig.get_config_var("EXT_SUFFIX") or ".so"


PYMOD = os.path.join(HERE, "flashtrie" + ext_suffix())


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True)
    out = "\n".join(l for l in p.stdout.splitlines()
                    if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError("build step failed: " + " ".join(cmd) + "\n" + out)
    return out


# Every file the libraries are built from: their sources and headers, the
# public headers, and this recipe (its flags).
def _source_files():
    files = [os.path.abspath(__file__)]
    for d in (CSRC, INC):
        for dirpath, dirnames, names in os.walk(d):
            dirnames[:] = sorted(x for x in dirnames if not x.startswith((".", "__")))
            files += [os.path.join(dirpath, n) for n in sorted(names)
                      if n.endswith((".h", ".hip", ".cpp", ".cc"))]
    return files


def source_id():
    """Build id of the current sources: sha256 (16 hex digits) over every
    source file's path (relative to the repository) and bytes.  Each built
    library carries the id of the sources it was built from."""
    h = hashlib.sha256()
    for f in _source_files():
        h.update(os.path.relpath(f, ROOT).encode() + b"\0")
        with open(f, "rb") as fh:
            h.update(fh.read())
        h.update(b"\0")
    return h.hexdigest()[:16]


ID_TAG = b"FT_BUILD_ID="


def built_id(path):
    """The build id embedded in a built library (None when absent)."""
    try:
        with open(path, "rb") as fh:
            data = fh.read()
    except OSError:
        return None
    i = data.find(ID_TAG)
    if i < 0:
        return None
    return data[i + len(ID_TAG):i + len(ID_TAG) + 16].decode("ascii", "replace")


def _pybind_includes():
    import pybind11
    return ["-I" + pybind11.get_include(),
            "-I" + sysconfig.get_paths()["include"]]


def build(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    bid = ["-DFT_BUILD_ID=\"" + source_id() + "\""]
    hip_objs = {
        "tbs_kernel.hip": os.path.join(OBJ, "tbs_kernel.o"),
        "ft_runtime.cpp": os.path.join(OBJ, "ft_runtime.o"),
    }
    host_objs = {
        "marisa_trie.cc": os.path.join(OBJ, "marisa_trie.o"),
        "image_builder.cc": os.path.join(OBJ, "image_builder.o"),
        "marisa_format.cc": os.path.join(OBJ, "marisa_format.o"),
        "topk_io.cc": os.path.join(OBJ, "topk_io.o"),
        "synth.cc": os.path.join(OBJ, "synth.o"),
        "synth_trie.cc": os.path.join(OBJ, "synth_trie.o"),
    }
    bind_obj = os.path.join(OBJ, "bindings.o")
    jobs = []
    for src, obj in hip_objs.items():
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        jobs.append([HIPCC] + HIP_FLAGS + bid + lang + ["-c", os.path.join(CSRC, src),
                                                        "-o", obj])
    for src, obj in host_objs.items():
        jobs.append([CXX] + CXX_FLAGS + bid + ["-c", os.path.join(CSRC, src),
                                               "-o", obj])
    jobs.append([HIPCC] + HIP_FLAGS + ["-x", "hip", os.path.join(CSRC, "copy_calib.hip"),
                                       "-o", COPY_CALIB])
    jobs.append([CXX] + CXX_FLAGS + bid + _pybind_includes() +
                ["-fvisibility=hidden", "-c", os.path.join(CSRC, "bindings.cc"),
                 "-o", bind_obj])
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        outs = list(ex.map(_run, jobs))
    if verbose:
        for o in outs:
            if o.strip():
                print(o)
    _run([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", LIB_AMD]
         + list(hip_objs.values()))
    _run([CXX, "-shared", "-fPIC", "-fopenmp", "-o", LIB_MARISA]
         + list(host_objs.values()) +
         ["-L" + HERE, "-lflashtrie_amd", "-Wl,-rpath,$ORIGIN"])
    # the beam-search command line tool (tools/marisa-beam-search.cc)
    _run([CXX] + CXX_FLAGS + [os.path.join(CSRC, "ft_beam_search.cc"), "-o", BEAM_CLI,
                              "-L" + HERE, "-lmarisa_amd", "-lflashtrie_amd",
                              "-Wl,-rpath,$ORIGIN"])
    _run([CXX, "-shared", "-fPIC", "-fopenmp", "-o", PYMOD, bind_obj,
          "-L" + HERE, "-lmarisa_amd", "-lflashtrie_amd",
          "-Wl,-rpath,$ORIGIN"])
    return [LIB_AMD, LIB_MARISA, PYMOD, COPY_CALIB, BEAM_CLI]


def built():
    """True when the three libraries exist and were built from the current
    sources (their embedded build ids equal source_id()); a stale build is
    rebuilt, never loaded."""
    sid = source_id()
    return all(built_id(p) == sid for p in (LIB_AMD, LIB_MARISA, PYMOD))


if __name__ == "__main__":
    for p in build(verbose="-v" in sys.argv):
        print(p)
