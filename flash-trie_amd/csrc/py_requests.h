// py_requests.h -- Python request arguments to ft_request rows and results
// to Python lists, for the `flashtrie` module's search entry points.
//
// The reference module takes beams / topk_id / topk_logp as nested Python
// lists converted by pybind11's generic STL casters
// (tools/bindings.cpp:45-119), which build one std::vector per row.  Here
// the same arguments are read in place:
//   * a numpy array (the whole batch [B][T][K], one request [T][K] or one
//     row [K]) whose dtype converts safely is used through the buffer
//     protocol, without a copy when it is already uint32 / float32 and
//     C-contiguous;
//   * a list or tuple of Python ints / floats is read with the CPython API
//     straight into one flat buffer per request;
//   * anything else (numpy scalars, bools, objects with __index__ or
//     __float__) goes through pybind11's own casters, so whatever the
//     reference's signature accepts is accepted and converts to the same
//     value, and whatever it rejects raises TypeError.
// Shape errors are those of marisa::Trie's checks (marisa_trie.cc
// check_shape), with the same messages.
#pragma once

#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/flashtrie_amd.h"
#include "marisa.h"

namespace ftpy {

namespace py = pybind11;

// One request's inputs, in C++ memory or in an array the caller holds.
struct ReqIn {
  std::vector<uint32_t> beams;
  size_t T = 0, K = 0;
  uint32_t F = 0;                    // final beam width (0: no search)
  std::vector<uint32_t> ids;         // [T * K] rows read from Python objects
  std::vector<float> lps;
  std::vector<const uint32_t*> id_rows;
  std::vector<const float*> lp_rows;
};

struct BadType {};  // the fast path cannot read an element: use pybind11's

// A Python int in [0, 2^32).  CPython 3.10 ints are sign-magnitude arrays
// of 30-bit digits (Py_SIZE = signed digit count), read here without a
// call; other versions use PyLong_AsUnsignedLong.
inline bool int_u32(PyObject* o, uint32_t* v) {
  if (!PyLong_CheckExact(o)) return false;
#if PY_VERSION_HEX < 0x030C0000 && PYLONG_BITS_IN_DIGIT == 30
  const Py_ssize_t n = Py_SIZE(o);
  const digit* d = ((PyLongObject*)o)->ob_digit;
  if (n == 0) {
    *v = 0;
    return true;
  }
  if (n == 1) {
    *v = (uint32_t)d[0];
    return true;
  }
  if (n == 2) {
    const uint64_t x = (uint64_t)d[0] | ((uint64_t)d[1] << 30);
    if (x >> 32) return false;
    *v = (uint32_t)x;
    return true;
  }
  return false;
#else
  const unsigned long x = PyLong_AsUnsignedLong(o);
  if (x == (unsigned long)-1 && PyErr_Occurred()) {
    PyErr_Clear();
    return false;
  }
  if ((uint64_t)x >> 32) return false;
  *v = (uint32_t)x;
  return true;
#endif
}

// A Python float (or int) as float: the double rounded to float, as
// pybind11's float caster does.
inline bool num_f32(PyObject* o, float* v) {
  if (PyFloat_CheckExact(o)) {
    *v = (float)PyFloat_AS_DOUBLE(o);
    return true;
  }
  if (PyLong_CheckExact(o)) {
    const double d = PyLong_AsDouble(o);
    if (d == -1.0 && PyErr_Occurred()) {
      PyErr_Clear();
      return false;
    }
    *v = (float)d;
    return true;
  }
  return false;
}

inline bool is_list_like(PyObject* o) { return PyList_CheckExact(o) || PyTuple_CheckExact(o); }

// `h` (a numpy array) as a C-contiguous array of T, or a null handle when
// its dtype does not convert safely.  Floating arrays of any width convert
// to float32 (numpy rounds to nearest like the C cast pybind11's float
// caster does); integer arrays only when every value is representable.
// (py::array's default constructor makes an empty array, not a null
// handle: the result is a py::object, null when there is no array.)
template <typename T>
py::object as_array(py::handle h) {
  if (!py::isinstance<py::array>(h)) return py::object();
  py::array src = py::reinterpret_borrow<py::array>(h);
  py::object out;
  const char kind = src.dtype().kind();
  if (std::is_same<T, float>::value && kind == 'f') {
    out = py::array_t<T, py::array::c_style | py::array::forcecast>::ensure(src);
  } else if (std::is_same<T, uint32_t>::value && (kind == 'i' || kind == 'u') &&
             !src.dtype().is(py::dtype::of<uint32_t>())) {
    // wider or signed integers: converted when every value is in [0, 2^32)
    // (pybind11's caster rejects the others, element by element)
    auto conv = [&](auto tag) -> py::object {
      using W = decltype(tag);
      auto w = py::array_t<W, py::array::c_style>::ensure(src);
      if (!w) {
        PyErr_Clear();
        return py::object();
      }
      std::vector<py::ssize_t> shape(w.shape(), w.shape() + w.ndim());
      py::array_t<uint32_t> o(shape);
      const W* a = w.data();
      uint32_t* b = o.mutable_data();
      for (py::ssize_t i = 0, n = w.size(); i < n; ++i) {
        if (a[i] < 0 || (uint64_t)a[i] > 0xFFFFFFFFull) return py::object();
        b[i] = (uint32_t)a[i];
      }
      return std::move(o);
    };
    out = kind == 'u' && src.dtype().itemsize() == 8 ? conv(uint64_t{}) : conv(int64_t{});
  } else {
    out = py::array_t<T, py::array::c_style>::ensure(src);
  }
  if (!out) PyErr_Clear();
  return out;
}

inline Py_ssize_t seq_len(py::handle h) {
  const Py_ssize_t n = PySequence_Size(h.ptr());
  if (n < 0) throw py::error_already_set();
  return n;
}

// Reads row object `row` (K elements) into out[K]: a list / tuple of
// Python numbers, or a 1-D numpy array.  BadType when an element is not a
// plain int / float or the array's dtype does not convert safely.
template <typename T>
void read_row(PyObject* row, size_t K, T* out, const char* what, size_t t) {
  auto ragged = [&]() {
    throw marisa::Exception(MARISA_CODE_ERROR,
                            "tbs: ragged topk rows (row " + std::to_string(t) + ")");
  };
  (void)what;
  if (is_list_like(row)) {
    if ((size_t)PySequence_Fast_GET_SIZE(row) != K) ragged();
    PyObject** it = PySequence_Fast_ITEMS(row);
    for (size_t k = 0; k < K; ++k) {
      bool ok;
      if constexpr (std::is_same<T, uint32_t>::value) ok = int_u32(it[k], out + k);
      else ok = num_f32(it[k], out + k);
      if (!ok) throw BadType();
    }
    return;
  }
  if (py::isinstance<py::array>(row)) {
    // safe casts only: an array pybind11 would convert element by element
    // to other values (or reject) takes the generic path
    py::object ao = as_array<T>(row);
    if (!ao) throw BadType();
    py::array a = py::reinterpret_borrow<py::array>(ao);
    if (a.ndim() != 1) throw BadType();
    if ((size_t)a.shape(0) != K) ragged();
    std::memcpy(out, a.data(), K * sizeof(T));
    return;
  }
  throw BadType();
}

// Reads one request's arguments into `q`: rows [0, T) in q.ids / q.lps, or
// pointing into topk_id / topk_logp when they are whole 2-D arrays (then
// appended to `keep`, which the caller holds until the search is done).
// Applies marisa::Trie's shape checks.
inline void read_request(py::handle beams, py::handle ids, py::handle lps, ReqIn& q,
                         std::vector<py::object>& keep) {
  // beams: a short list; pybind11's caster keeps its exact semantics
  q.beams = py::cast<std::vector<uint32_t>>(beams);
  q.T = q.K = 0;
  q.F = 0;
  if (q.beams.empty()) throw marisa::Exception(MARISA_CODE_ERROR, "tbs: beams is empty");
  q.F = q.beams.back();
  if (q.F == 0) {
    // no search and no shape checks (outputs stay empty), but the rows are
    // still converted, as the reference's signature does
    throw BadType();
  }
  const size_t T = (size_t)seq_len(lps);
  const size_t nid = (size_t)seq_len(ids);
  if (T == 0 || nid == 0) throw marisa::Exception(MARISA_CODE_ERROR, "tbs: topk rows are empty");
  // whole [T'][K] arrays: rows point into them (T' >= T rows of ids)
  const py::object aio = as_array<uint32_t>(ids), alo = as_array<float>(lps);
  const bool whole_i = aio && py::reinterpret_borrow<py::array>(aio).ndim() == 2;
  const bool whole_l = alo && py::reinterpret_borrow<py::array>(alo).ndim() == 2;
  const uint32_t* ai = nullptr;
  const float* al = nullptr;
  size_t K, Kl = 0;
  if (whole_l) {
    const py::array a = py::reinterpret_borrow<py::array>(alo);
    al = (const float*)a.data();
    Kl = (size_t)a.shape(1);
  }
  if (whole_i) {
    const py::array a = py::reinterpret_borrow<py::array>(aio);
    ai = (const uint32_t*)a.data();
    K = (size_t)a.shape(1);
  } else {
    py::object row0 = py::reinterpret_steal<py::object>(PySequence_GetItem(ids.ptr(), 0));
    if (!row0) throw py::error_already_set();
    K = (size_t)seq_len(row0);
  }
  if (K == 0) throw marisa::Exception(MARISA_CODE_ERROR, "tbs: topk row 0 is empty");
  if (nid < T)
    throw marisa::Exception(MARISA_CODE_ERROR, "tbs: fewer topk_id rows than topk_logp rows");
  if (q.beams.size() < T)
    throw marisa::Exception(MARISA_CODE_ERROR, "tbs: fewer beam widths than steps");
  for (size_t t = 0; t < T; ++t)
    if (q.beams[t] == 0)
      throw marisa::Exception(MARISA_CODE_ERROR, "tbs: beam width 0 at step " + std::to_string(t));
  q.T = T;
  q.K = K;
  q.id_rows.resize(T);
  q.lp_rows.resize(T);
  if (whole_l && Kl != K)
    throw marisa::Exception(MARISA_CODE_ERROR, "tbs: ragged topk rows (row 0)");
  if (!whole_i) q.ids.resize(T * K);
  if (!whole_l) q.lps.resize(T * K);
  for (size_t t = 0; t < T; ++t) {
    if (whole_i) {
      q.id_rows[t] = ai + t * K;
    } else {
      PyObject* r = is_list_like(ids.ptr()) ? PySequence_Fast_GET_ITEM(ids.ptr(), t) : nullptr;
      py::object hold;
      if (!r) {
        hold = py::reinterpret_steal<py::object>(PySequence_GetItem(ids.ptr(), (Py_ssize_t)t));
        if (!hold) throw py::error_already_set();
        r = hold.ptr();
      }
      read_row<uint32_t>(r, K, q.ids.data() + t * K, "topk_id", t);
      q.id_rows[t] = q.ids.data() + t * K;
    }
    if (whole_l) {
      q.lp_rows[t] = al + t * K;
    } else {
      PyObject* r = is_list_like(lps.ptr()) ? PySequence_Fast_GET_ITEM(lps.ptr(), t) : nullptr;
      py::object hold;
      if (!r) {
        hold = py::reinterpret_steal<py::object>(PySequence_GetItem(lps.ptr(), (Py_ssize_t)t));
        if (!hold) throw py::error_already_set();
        r = hold.ptr();
      }
      read_row<float>(r, K, q.lps.data() + t * K, "topk_logp", t);
      q.lp_rows[t] = q.lps.data() + t * K;
    }
  }
  if (whole_i) keep.push_back(aio);
  if (whole_l) keep.push_back(alo);
}

// The generic path: pybind11's casters (the reference's), then the same
// flat layout.  Raises TypeError for what they reject.
inline void read_request_generic(py::handle beams, py::handle ids, py::handle lps, ReqIn& q) {
  std::vector<uint32_t> b;
  std::vector<std::vector<uint32_t>> vi;
  std::vector<std::vector<float>> vl;
  try {
    b = py::cast<std::vector<uint32_t>>(beams);
    vi = py::cast<std::vector<std::vector<uint32_t>>>(ids);
    vl = py::cast<std::vector<std::vector<float>>>(lps);
  } catch (const py::cast_error&) {
    throw py::type_error(
        "incompatible arguments: beams must be a sequence of ints, topk_id a sequence of "
        "rows of ints in [0, 2^32), topk_logp a sequence of rows of floats");
  }
  q.beams = b;
  q.T = q.K = 0;
  q.F = 0;
  if (b.empty()) throw marisa::Exception(MARISA_CODE_ERROR, "tbs: beams is empty");
  q.F = b.back();
  if (q.F == 0) return;
  const size_t T = vl.size();
  if (T == 0 || vi.empty()) throw marisa::Exception(MARISA_CODE_ERROR, "tbs: topk rows are empty");
  const size_t K = vi[0].size();
  if (K == 0) throw marisa::Exception(MARISA_CODE_ERROR, "tbs: topk row 0 is empty");
  if (vi.size() < T)
    throw marisa::Exception(MARISA_CODE_ERROR, "tbs: fewer topk_id rows than topk_logp rows");
  if (b.size() < T)
    throw marisa::Exception(MARISA_CODE_ERROR, "tbs: fewer beam widths than steps");
  q.T = T;
  q.K = K;
  q.ids.resize(T * K);
  q.lps.resize(T * K);
  q.id_rows.resize(T);
  q.lp_rows.resize(T);
  for (size_t t = 0; t < T; ++t) {
    if (vi[t].size() != K || vl[t].size() != K)
      throw marisa::Exception(MARISA_CODE_ERROR,
                              "tbs: ragged topk rows (row " + std::to_string(t) + ")");
    if (b[t] == 0)
      throw marisa::Exception(MARISA_CODE_ERROR, "tbs: beam width 0 at step " + std::to_string(t));
    std::memcpy(q.ids.data() + t * K, vi[t].data(), K * 4);
    std::memcpy(q.lps.data() + t * K, vl[t].data(), K * 4);
    q.id_rows[t] = q.ids.data() + t * K;
    q.lp_rows[t] = q.lps.data() + t * K;
  }
}

inline void read_any(py::handle beams, py::handle ids, py::handle lps, ReqIn& q,
                     std::vector<py::object>& keep) {
  try {
    read_request(beams, ids, lps, q, keep);
  } catch (const BadType&) {
    read_request_generic(beams, ids, lps, q);
  } catch (const py::cast_error&) {
    read_request_generic(beams, ids, lps, q);
  }
}

// Item i of a batch argument (a list / tuple of requests or a numpy array
// with one more dimension).
inline py::object batch_item(py::handle seq, size_t i) {
  PyObject* o = PySequence_GetItem(seq.ptr(), (Py_ssize_t)i);
  if (!o) throw py::error_already_set();
  return py::reinterpret_steal<py::object>(o);
}

// One request's results as (list of token lists, list of norms).
// Holds the cyclic garbage collector off while a call builds its result
// lists, and restores its state after.  A batch's results are ~700 lists,
// enough to cross the collector's young-generation threshold inside the
// call, and a collection there traverses every young container -- above
// all the caller's input rows, alive and young during the call (a batch of
// 8 x 16 rows of 1000 as .tolist() lists: 256K items, ~0.35 ms a
// collection).  Deferred, the count is balanced again when the caller
// drops its lists and results, as it is without a search.  Lists of ints
// form no cycles, so nothing the collector would free is kept.
class GcPause {
 public:
  GcPause() : was_(PyGC_Disable()) {}
  ~GcPause() {
    if (was_) PyGC_Enable();
  }
  GcPause(const GcPause&) = delete;
  GcPause& operator=(const GcPause&) = delete;

 private:
  int was_;
};

inline std::pair<py::object, py::object> result_lists(const ft_result& r) {
  const uint32_t n = r.count;
  py::object sents = py::reinterpret_steal<py::object>(PyList_New(n));
  py::object norms = py::reinterpret_steal<py::object>(PyList_New(n));
  if (!sents || !norms) throw py::error_already_set();
  for (uint32_t j = 0; j < n; ++j) {
    const uint32_t len = r.length[j];
    const uint32_t* tk = r.tokens + (size_t)j * r.token_stride;
    PyObject* s = PyList_New(len);
    if (!s) throw py::error_already_set();
    PyList_SET_ITEM(sents.ptr(), j, s);
    for (uint32_t k = 0; k < len; ++k) {
      PyObject* v = PyLong_FromUnsignedLong(tk[k]);
      if (!v) throw py::error_already_set();
      PyList_SET_ITEM(s, k, v);
    }
    PyObject* f = PyFloat_FromDouble(r.logp_norm[j]);
    if (!f) throw py::error_already_set();
    PyList_SET_ITEM(norms.ptr(), j, f);
  }
  return {sents, norms};
}

}  // namespace ftpy
