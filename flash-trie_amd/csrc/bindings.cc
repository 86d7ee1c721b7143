// bindings.cc -- the `flashtrie` Python module.
//
// Same names, arguments, defaults and return shapes as the reference module
// (tools/bindings.cpp:24-122): Trie (load, mmap, build, total_size,
// num_tries, num_keys, num_nodes, save, clear, init_tbs_gpu), tbs,
// bs_tbs_gpu and load_topk_keys_and_scores.  Errors raise RuntimeError.
//
// Beyond the reference: numpy entry points used by the benchmark and tests
// (build_arrays, image, stage / launch / sync / fetch, search_np) and the
// seeded synthetic generators (synth_keys, synth_requests).
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <chrono>
#include <cstring>
#include <fstream>
#include <functional>
#include <iostream>
#include <numeric>
#include <sstream>
#include <thread>

#include "../../include/flashtrie_amd.h"
#include "image_builder.h"
#include "marisa_format.h"
#include "marisa.h"
#include "marisa/topk_io.h"
#include "py_requests.h"
#include "synth.h"
#include "trie_impl.h"

namespace py = pybind11;
// u64 per step of ft_result::step_stats (include/flashtrie_amd.h)
constexpr size_t ftk_step_stats = FT_STEP_STATS;
using marisa::Label;
using marisa::TbsInput;
using marisa::Trie;


namespace {

ft_ctx* ctx_of(const Trie& t) {
  marisa::TrieImpl* im = t.impl();
  if (!im || !im->ctx)
    throw marisa::Exception(MARISA_STATE_ERROR, "init_tbs_gpu was not called");
  return im->ctx;
}

const ftamd::ImageBlob& image_of(const Trie& t) {
  marisa::TrieImpl* im = t.impl();
  if (!im || im->img.empty())
    throw marisa::Exception(MARISA_STATE_ERROR, "trie is not built or loaded");
  return im->img;
}

void check_ft(int rc, const char* where) {
  if (rc == FT_OK) return;
  std::string msg = std::string(where) + ": " + ft_strerror(rc);
  const char* d = ft_last_error();
  if (d && *d) msg += std::string(" (") + d + ")";
  throw marisa::Exception(MARISA_STATE_ERROR, msg);
}

// --- numpy batch staging (benchmark path) ----------------------------------
struct NpBatch {
  std::vector<ft_request> reqs;
  std::vector<uint32_t> F, T;
  uint32_t K = 0;
};

NpBatch& staged_batch() {
  static NpBatch b;
  return b;
}

// Error of a search, as Trie::tbs_gpu_batched raises it.
[[noreturn]] void throw_search(int rc) {
  std::string msg = std::string("tbs_gpu_batched: ") + ft_strerror(rc);
  const char* d = ft_last_error();
  if (d && *d) msg += std::string(" (") + d + ")";
  marisa::ErrorCode code = MARISA_STATE_ERROR;
  if (rc == FT_E_ARG || rc == FT_E_INPUT) code = MARISA_CODE_ERROR;
  if (rc == FT_E_LIMIT) code = MARISA_SIZE_ERROR;
  if (rc == FT_E_NOMEM) code = MARISA_MEMORY_ERROR;
  throw marisa::Exception(code, msg);
}

// The GPU search behind bs_tbs_gpu and tbs(use_gpu=True): B requests,
// either one request's (beams, topk_id, topk_logp) handles or the three
// batch arguments (`batch`, each indexable by request).  Inputs are read
// in place (py_requests.h) with the GIL held; the search runs without it;
// the results become Python lists.  Returns (out_sent, out_logp_norm, ms,
// phase) like the reference's bs_tbs_gpu: ms is timed from the inputs
// being in C++ memory to the results being there, as the reference times
// it (tools/bindings.cpp:90-100), and phase holds per request [expansion,
// validation, selection, overhead, kernel] device ms.
py::tuple gpu_search(Trie& trie, size_t B, const py::object* one_beams,
                     const py::object* one_ids, const py::object* one_lps,
                     const py::handle* batch, float tok_thr, double sent_thr, double alpha,
                     bool early) {
  ft_ctx* c = ctx_of(trie);
  marisa::TrieImpl* im = trie.impl();
  // per-thread buffers (the GIL is released during the search, so another
  // thread may convert its own call meanwhile)
  struct Buf {
    std::vector<ftpy::ReqIn> in;
    std::vector<ft_request> reqs;
    std::vector<ft_result> res;
    std::vector<std::vector<double>> norms;
    std::vector<std::vector<uint32_t>> lens, toks;
  };
  static thread_local Buf b;
  if (b.in.size() < B) {
    b.in.resize(B);
    b.norms.resize(B);
    b.lens.resize(B);
    b.toks.resize(B);
  }
  b.reqs.assign(B, ft_request{});
  b.res.assign(B, ft_result{});
  std::vector<py::object> keep;
  for (size_t i = 0; i < B; ++i) {
    ftpy::ReqIn& q = b.in[i];
    if (batch) {
      const py::object bi = ftpy::batch_item(batch[0], i), ii = ftpy::batch_item(batch[1], i),
                       li = ftpy::batch_item(batch[2], i);
      ftpy::read_any(bi, ii, li, q, keep);
    } else {
      ftpy::read_any(*one_beams, *one_ids, *one_lps, q, keep);
    }
    ft_request& r = b.reqs[i];
    r.beams = q.beams.data();
    r.num_beams = (uint32_t)q.beams.size();
    r.token_logp_threshold = tok_thr;
    r.sent_logp_threshold = sent_thr;
    r.length_norm = alpha;
    r.early_exit = early ? 1 : 0;
    if (q.F == 0) continue;  // outputs untouched
    r.num_steps = (uint32_t)q.T;
    r.topk = (uint32_t)q.K;
    r.topk_id_rows = q.id_rows.data();
    r.topk_logp_rows = q.lp_rows.data();
    // result arrays, grown as needed and never shrunk
    if (b.norms[i].size() < q.F) b.norms[i].resize(q.F);
    if (b.lens[i].size() < q.F) b.lens[i].resize(q.F);
    if (b.toks[i].size() < (size_t)q.F * q.T) b.toks[i].resize((size_t)q.F * q.T);
    ft_result& o = b.res[i];
    o.capacity = q.F;
    o.token_stride = (uint32_t)q.T;
    o.logp_norm = b.norms[i].data();
    o.length = b.lens[i].data();
    o.tokens = b.toks[i].data();
  }
  using clk = std::chrono::high_resolution_clock;
  const auto start = clk::now();
  int rc;
  {
    py::gil_scoped_release nogil;
    std::lock_guard<std::mutex> lock(im->search_mu);
    rc = ft_search(c, b.reqs.data(), B, b.res.data(), nullptr);
  }
  const auto end = clk::now();
  if (rc) throw_search(rc);
  ftpy::GcPause no_gc;
  py::list sents(B), norms(B), phase(B);
  for (size_t i = 0; i < B; ++i) {
    const ft_result& o = b.res[i];
    if (b.in[i].F) {
      auto sl = ftpy::result_lists(o);
      sents[i] = std::move(sl.first);
      norms[i] = std::move(sl.second);
    } else {
      sents[i] = py::list();
      norms[i] = py::list();
    }
    phase[i] = py::cast(std::vector<double>{o.device_ms[0], 0.0, o.device_ms[1],
                                            o.device_ms[2], o.device_ms[3]});
  }
  return py::make_tuple(sents, norms, marisa::get_msec(start, end), phase);
}

}  // namespace

#ifndef FT_BUILD_ID
#define FT_BUILD_ID "unknown"
#endif
// the build id tag of this module (see ft_build_id)
extern "C" __attribute__((used, visibility("default"))) const char ft_module_build_id[] =
    "FT_BUILD_ID=" FT_BUILD_ID;

PYBIND11_MODULE(flashtrie, m) {
  m.doc() = "MI355X trie beam search (drop-in for the reference flashtrie module)";
  // the build ids of this module and of the C ABI library it loaded: the
  // same unless a library was rebuilt alone
  m.def("build_id", []() {
    if (std::strcmp(ft_build_id(), ft_module_build_id + 12) != 0)
      throw marisa::Exception(MARISA_STATE_ERROR,
                              std::string("build_id: the module (") + (ft_module_build_id + 12) +
                                  ") and libflashtrie_amd.so (" + ft_build_id() +
                                  ") come from different builds");
    return std::string(ft_build_id());
  });
  py::register_exception<marisa::Exception>(m, "MarisaError", PyExc_RuntimeError);

  py::class_<Trie>(m, "Trie")
      .def(py::init<>())
      // a MARISA trie.bin written by the reference, or an image from save()
      .def("load",
           [](Trie& t, const std::string& p) {
             py::gil_scoped_release nogil;
             t.load(p.c_str());
           })
      .def("mmap",
           [](Trie& t, const std::string& p) {
             py::gil_scoped_release nogil;
             t.mmap(p.c_str());
           })
      .def("build",
           [](Trie& t, const std::vector<std::vector<uint32_t>>& rows) {
             marisa::Keyset ks;
             for (const auto& r : rows) ks.push_back(r.data(), r.size());
             t.build(ks, 1 | MARISA_TEXT_TAIL | MARISA_LABEL_ORDER | MARISA_DEFAULT_CACHE);
           },
           py::arg("token_rows"))
      // beyond the reference module (its C++ Trie has them,
      // lib/marisa/trie.cc:33-43, 57-67, 78-86): a trie from a buffer used
      // in place (kept alive with the Trie), or from / to a descriptor
      .def(
          "map",
          [](Trie& t, py::buffer b) {
            py::buffer_info bi = b.request();
            const size_t n = (size_t)bi.size * (size_t)bi.itemsize;
            if (bi.ndim > 1 && !(bi.strides.back() == bi.itemsize))
              throw marisa::Exception(MARISA_CODE_ERROR, "map: the buffer must be contiguous");
            py::gil_scoped_release nogil;
            t.map(bi.ptr, n);
          },
          py::arg("buffer"), py::keep_alive<1, 2>())
      .def("read",
           [](Trie& t, int fd) {
             py::gil_scoped_release nogil;
             t.read(fd);
           },
           py::arg("fd"))
      .def("write",
           [](const Trie& t, int fd) {
             py::gil_scoped_release nogil;
             t.write(fd);
           },
           py::arg("fd"))
      .def("total_size", &Trie::total_size)
      .def("num_tries", &Trie::num_tries)
      .def("num_keys", &Trie::num_keys)
      .def("num_nodes", &Trie::num_nodes)
      .def("save", [](const Trie& t, const std::string& p) { t.save(p.c_str()); })
      .def("save_marisa",
           [](const Trie& t, const std::string& p) {
             py::gil_scoped_release nogil;
             t.save_marisa(p.c_str());
           })
      .def("clear", &Trie::clear)
      .def("get_max_batch_size", &Trie::get_max_batch_size)
      .def("init_tbs_gpu", &Trie::init_tbs_gpu, py::arg("max_batch_size"),
           py::arg("max_num_topk") = 1024, py::arg("max_num_outpos") = 64,
           py::arg("max_num_out_beams") = 8192,
           py::arg("max_num_out_tokens") = 8192 * 64,
           py::arg("max_num_inter_beams") = 1024 * 1024,
           py::arg("radix_topk_threshold") = 1024)
      // ---- beyond the reference ----
      .def("build_arrays",
           [](Trie& t, py::array_t<uint32_t, py::array::c_style | py::array::forcecast> toks,
              py::array_t<uint64_t, py::array::c_style | py::array::forcecast> offs,
             bool progress) {
             if (offs.ndim() != 1 || offs.shape(0) < 1)
               throw marisa::Exception(MARISA_CODE_ERROR, "offsets must be 1-D, length >= 1");
             const uint64_t n = (uint64_t)offs.shape(0) - 1;
             const uint64_t* o = offs.data();
             if (o[0] != 0 || o[n] != (uint64_t)toks.size())
               throw marisa::Exception(MARISA_CODE_ERROR, "offsets do not cover the tokens");
             ftamd::ImageBlob img;
             std::string err;
             bool ok;
             {
               py::gil_scoped_release nogil;
               ok = ftamd::build_image_from_keys(toks.data(), o, n, &img, &err, 0, progress);
             }
             if (!ok) throw marisa::Exception(MARISA_SIZE_ERROR, "build: " + err);
             t.assign_image(img.data(), img.size());
           },
           py::arg("tokens"), py::arg("offsets"), py::arg("progress") = false)
      .def("image",
           [](const Trie& t) {
             const ftamd::ImageBlob& img = image_of(t);
             return py::array_t<uint8_t>((py::ssize_t)img.size(), img.data());
           })
      .def("image_view",
           [](py::object self) {
             // zero-copy view of the image; keeps the Trie alive
             const Trie& t = self.cast<const Trie&>();
             const ftamd::ImageBlob& img = image_of(t);
             return py::array_t<uint8_t>({(py::ssize_t)img.size()}, {(py::ssize_t)1},
                                         img.data(), self);
           })
      .def("marisa_bytes",
           [](const Trie& t) {
             // the MARISA trie file save_marisa writes
             std::vector<uint8_t> out;
             std::string err;
             if (!ftamd::marisa_from_image(image_of(t), &out, &err))
               throw marisa::Exception(MARISA_FORMAT_ERROR, "marisa_bytes: " + err);
             return py::array_t<uint8_t>((py::ssize_t)out.size(), out.data());
           })
      .def("load_marisa_bytes",
           [](Trie& t, py::array_t<uint8_t, py::array::c_style | py::array::forcecast> a) {
             // a MARISA trie file held in memory (lib/marisa/trie.cc:34-42)
             ftamd::ImageBlob img;
             std::string err;
             bool ok;
             {
               py::gil_scoped_release nogil;
               ok = ftamd::image_from_marisa(a.data(), (size_t)a.size(), &img, &err);
             }
             if (!ok) throw marisa::Exception(MARISA_FORMAT_ERROR, "load_marisa_bytes: " + err);
             t.assign_image(img.data(), img.size());
           },
           py::arg("data"))
      .def("assign_image",
           [](Trie& t, py::array_t<uint8_t, py::array::c_style | py::array::forcecast> a) {
             t.assign_image(a.data(), (size_t)a.size());
           })
      .def("device_info", [](const Trie& t) {
        int cus = 0, lds = 0, khz = 0;
        char name[64] = {0};
        check_ft(ft_device_info(ctx_of(t), &cus, &lds, &khz, name, sizeof(name)),
                 "device_info");
        py::dict d;
        d["num_cus"] = cus;
        d["lds_per_block"] = lds;
        d["wall_clock_khz"] = khz;
        d["arch"] = std::string(name);
        return d;
      });

  m.def(
      "tbs",
      [](Trie& trie, py::object beams, py::object topk_id, py::object topk_logp,
         float token_logp_threshold, double sent_logp_threshold, double length_norm,
         bool early_exit, bool use_gpu) -> py::tuple {
        if (use_gpu) {
          // one request through the batched path (Trie::tbs_gpu: batch slot 0)
          py::tuple r = gpu_search(trie, 1, &beams, &topk_id, &topk_logp, nullptr,
                                   token_logp_threshold, sent_logp_threshold, length_norm,
                                   early_exit);
          return py::make_tuple(py::reinterpret_borrow<py::list>(r[0])[0],
                                py::reinterpret_borrow<py::list>(r[1])[0], r[2]);
        }
        // the host search takes the reference's vectors
        ftpy::ReqIn q;
        std::vector<py::object> keep;
        ftpy::read_any(beams, topk_id, topk_logp, q, keep);
        std::vector<std::vector<Label>> vi(q.T), out_sent;
        std::vector<std::vector<float>> vl(q.T);
        for (size_t t = 0; t < q.T; ++t) {
          vi[t].assign(q.id_rows[t], q.id_rows[t] + q.K);
          vl[t].assign(q.lp_rows[t], q.lp_rows[t] + q.K);
        }
        std::vector<double> out_logp_norm;
        auto start = std::chrono::high_resolution_clock::now();
        TbsInput input{q.beams, vi, vl, out_sent, out_logp_norm, token_logp_threshold,
                       sent_logp_threshold, length_norm, early_exit};
        {
          py::gil_scoped_release nogil;
          if (q.F) trie.tbs(input);
        }
        auto end = std::chrono::high_resolution_clock::now();
        ftpy::GcPause no_gc;
        return py::make_tuple(py::cast(out_sent), py::cast(out_logp_norm),
                              marisa::get_msec(start, end));
      },
      py::arg("trie"), py::arg("beams"), py::arg("topk_id"), py::arg("topk_logp"),
      py::arg("token_logp_threshold"), py::arg("sents_logp_threshold"),
      py::arg("length_norm"), py::arg("early_exit"), py::arg("use_gpu") = false);

  m.def(
      "bs_tbs_gpu",
      [](Trie& trie, size_t batch_size, py::object batch_beams, py::object batch_topk_id,
         py::object batch_topk_logp, float token_logp_threshold, double sent_logp_threshold,
         double length_norm, bool early_exit) {
        ctx_of(trie);  // init_tbs_gpu must have run
        if (batch_size > trie.get_max_batch_size())
          throw marisa::Exception(MARISA_BOUND_ERROR, "bs_tbs_gpu: batch_size > max_batch_size");
        if (batch_size != (size_t)ftpy::seq_len(batch_topk_id) ||
            batch_size != (size_t)ftpy::seq_len(batch_topk_logp) ||
            batch_size != (size_t)ftpy::seq_len(batch_beams))
          throw marisa::Exception(MARISA_CODE_ERROR, "bs_tbs_gpu: batch_size does not match the inputs");
        return gpu_search(trie, batch_size, nullptr, nullptr, nullptr,
                          std::array<py::handle, 3>{batch_beams, batch_topk_id, batch_topk_logp}
                              .data(),
                          token_logp_threshold, sent_logp_threshold, length_norm, early_exit);
      },
      py::arg("trie"), py::arg("batch_size"), py::arg("batch_beams"),
      py::arg("batch_topk_id"), py::arg("batch_topk_logp"),
      py::arg("token_logp_threshold"), py::arg("sents_logp_threshold"),
      py::arg("length_norm"), py::arg("early_exit"));

  // The conversion of one request's arguments, as the search entry points
  // read them: (beams, ids[T][K], logps[T][K]), for tests on the CPU.
  m.def(
      "_convert_request",
      [](py::object beams, py::object topk_id, py::object topk_logp, bool generic) {
        ftpy::ReqIn q;
        std::vector<py::object> keep;
        if (generic) ftpy::read_request_generic(beams, topk_id, topk_logp, q);
        else ftpy::read_any(beams, topk_id, topk_logp, q, keep);
        py::array_t<uint32_t> ids({(py::ssize_t)q.T, (py::ssize_t)q.K});
        py::array_t<float> lps({(py::ssize_t)q.T, (py::ssize_t)q.K});
        for (size_t t = 0; t < q.T; ++t) {
          std::memcpy(ids.mutable_data() + t * q.K, q.id_rows[t], q.K * 4);
          std::memcpy(lps.mutable_data() + t * q.K, q.lp_rows[t], q.K * 4);
        }
        return py::make_tuple(py::cast(q.beams), ids, lps);
      },
      py::arg("beams"), py::arg("topk_id"), py::arg("topk_logp"), py::arg("generic") = false);

  // result_lists on caller-made results (tests): lengths[n], tokens[n, T]
  m.def(
      "_result_lists",
      [](py::array_t<uint32_t, py::array::c_style | py::array::forcecast> lengths,
         py::array_t<uint32_t, py::array::c_style | py::array::forcecast> tokens,
         py::array_t<double, py::array::c_style | py::array::forcecast> norms) {
        if (tokens.ndim() != 2 || lengths.ndim() != 1 || norms.ndim() != 1 ||
            lengths.shape(0) != tokens.shape(0) || norms.shape(0) != tokens.shape(0))
          throw py::value_error("_result_lists: lengths[n], tokens[n, T], norms[n]");
        ft_result r{};
        r.capacity = r.count = (uint32_t)tokens.shape(0);
        r.token_stride = (uint32_t)tokens.shape(1);
        for (py::ssize_t j = 0; j < lengths.shape(0); ++j)
          if (lengths.data()[j] > r.token_stride) throw py::value_error("_result_lists: length");
        r.length = const_cast<uint32_t*>(lengths.data());
        r.tokens = const_cast<uint32_t*>(tokens.data());
        r.logp_norm = const_cast<double*>(norms.data());
        ftpy::GcPause no_gc;
        auto sl = ftpy::result_lists(r);
        return py::make_tuple(sl.first, sl.second);
      },
      py::arg("lengths"), py::arg("tokens"), py::arg("norms"));

  m.def("load_topk_keys_and_scores", &marisa::load_topk_keys_and_scores,
        py::arg("dataset_dir"));

  // ---- the reference's timing boundary, driven from C++ ----------------------
  m.def(
      "bench_boundary",
      [](Trie& trie, py::array_t<uint32_t, py::array::c_style | py::array::forcecast> beams,
         py::array_t<uint32_t, py::array::c_style | py::array::forcecast> ids,
         py::array_t<float, py::array::c_style | py::array::forcecast> logp, size_t batch,
         float token_logp_threshold, double sent_logp_threshold, double length_norm,
         bool early_exit, int warmup_passes, int passes) {
        // Consecutive batches of `batch` requests, each converted to
        // TbsInput vectors (untimed, as the module converts Python lists
        // before its timer) and searched by Trie::tbs_gpu_batched; the call
        // is timed with steady_clock exactly where bs_tbs_gpu times it
        // (tools/bindings.cpp:90-100): staging, H2D, the launch, D2H and the
        // filled output vectors.  Returns (call_ms[passes][calls],
        // pass_s[passes] -- wall time of each measured pass, conversions
        // included -- and, for every request of the last pass, its result
        // count and an FNV-1a hash over 32-bit words of (count, then per
        // result: length, tokens, the two words of the norm)).
        if (beams.ndim() != 2 || ids.ndim() != 3 || logp.ndim() != 3 ||
            ids.shape(0) != beams.shape(0) || ids.shape(1) != beams.shape(1) ||
            logp.shape(0) != ids.shape(0) || logp.shape(1) != ids.shape(1) ||
            logp.shape(2) != ids.shape(2))
          throw marisa::Exception(MARISA_CODE_ERROR,
                                  "bench_boundary: shapes must be [n][T], [n][T][K]");
        if (batch == 0 || passes < 1 || warmup_passes < 0)
          throw marisa::Exception(MARISA_CODE_ERROR, "bench_boundary: bad batch or passes");
        const size_t n = beams.shape(0), T = beams.shape(1), K = ids.shape(2);
        const size_t calls = n / batch;
        if (calls == 0)
          throw marisa::Exception(MARISA_CODE_ERROR, "bench_boundary: fewer requests than batch");
        py::array_t<double> call_ms({(py::ssize_t)passes, (py::ssize_t)calls});
        py::array_t<double> pass_s((py::ssize_t)passes);
        py::array_t<uint32_t> counts((py::ssize_t)(calls * batch));
        py::array_t<uint64_t> hashes((py::ssize_t)(calls * batch));
        const uint32_t* bp = beams.data();
        const uint32_t* ip = ids.data();
        const float* lp = logp.data();
        double* cm = call_ms.mutable_data();
        double* ps = pass_s.mutable_data();
        uint32_t* cp = counts.mutable_data();
        uint64_t* hp = hashes.mutable_data();
        {
          py::gil_scoped_release nogil;
          using clk = std::chrono::steady_clock;
          std::vector<std::vector<uint32_t>> bb(batch);
          std::vector<std::vector<std::vector<Label>>> tid(batch);
          std::vector<std::vector<std::vector<float>>> tlp(batch);
          std::vector<std::vector<std::vector<Label>>> out_sent(batch);
          std::vector<std::vector<double>> out_norm(batch);
          for (int p = 0; p < warmup_passes + passes; ++p) {
            const bool measured = p >= warmup_passes;
            const auto p0 = clk::now();
            for (size_t c = 0; c < calls; ++c) {
              std::vector<TbsInput> inputs;
              inputs.reserve(batch);
              for (size_t i = 0; i < batch; ++i) {
                const size_t r = c * batch + i;
                bb[i].assign(bp + r * T, bp + (r + 1) * T);
                tid[i].resize(T);
                tlp[i].resize(T);
                for (size_t t = 0; t < T; ++t) {
                  tid[i][t].assign(ip + (r * T + t) * K, ip + (r * T + t + 1) * K);
                  tlp[i][t].assign(lp + (r * T + t) * K, lp + (r * T + t + 1) * K);
                }
                out_sent[i].clear();
                out_norm[i].clear();
                inputs.push_back(TbsInput{bb[i], tid[i], tlp[i], out_sent[i], out_norm[i],
                                          token_logp_threshold, sent_logp_threshold,
                                          length_norm, early_exit});
              }
              const auto t0 = clk::now();
              trie.tbs_gpu_batched(inputs);
              const auto t1 = clk::now();
              if (measured)
                cm[(size_t)(p - warmup_passes) * calls + c] =
                    std::chrono::duration<double, std::milli>(t1 - t0).count();
              if (p == warmup_passes + passes - 1) {
                for (size_t i = 0; i < batch; ++i) {
                  uint64_t h = 0xcbf29ce484222325ull;
                  auto mix = [&h](uint32_t w) {
                    h ^= w;
                    h *= 0x100000001b3ull;
                  };
                  const auto& os = out_sent[i];
                  mix((uint32_t)os.size());
                  for (size_t j = 0; j < os.size(); ++j) {
                    mix((uint32_t)os[j].size());
                    for (Label tk : os[j]) mix(tk);
                    uint64_t bits;
                    std::memcpy(&bits, &out_norm[i][j], 8);
                    mix((uint32_t)bits);
                    mix((uint32_t)(bits >> 32));
                  }
                  cp[c * batch + i] = (uint32_t)os.size();
                  hp[c * batch + i] = h;
                }
              }
            }
            if (measured)
              ps[p - warmup_passes] =
                  std::chrono::duration<double>(clk::now() - p0).count();
          }
        }
        return py::make_tuple(call_ms, pass_s, counts, hashes);
      },
      py::arg("trie"), py::arg("beams"), py::arg("topk_id"), py::arg("topk_logp"),
      py::arg("batch"), py::arg("token_logp_threshold"), py::arg("sents_logp_threshold"),
      py::arg("length_norm"), py::arg("early_exit"), py::arg("warmup_passes") = 1,
      py::arg("passes") = 2);

  // ---- numpy batch path: stage / launch / sync / fetch -----------------------
  m.def(
      "stage",
      [](Trie& trie, py::array_t<uint32_t, py::array::c_style | py::array::forcecast> beams,
         py::array_t<uint32_t, py::array::c_style | py::array::forcecast> ids,
         py::array_t<float, py::array::c_style | py::array::forcecast> logp,
         float token_logp_threshold, double sent_logp_threshold, double length_norm,
         bool early_exit) {
        // beams [B][T], ids / logp [B][T][K]
        if (beams.ndim() != 2 || ids.ndim() != 3 || logp.ndim() != 3 ||
            ids.shape(0) != beams.shape(0) || ids.shape(1) != beams.shape(1) ||
            logp.shape(0) != ids.shape(0) || logp.shape(1) != ids.shape(1) ||
            logp.shape(2) != ids.shape(2))
          throw marisa::Exception(MARISA_CODE_ERROR, "stage: shapes must be [B][T], [B][T][K]");
        ft_ctx* c = ctx_of(trie);
        NpBatch& nb = staged_batch();
        const size_t B = beams.shape(0), T = beams.shape(1), K = ids.shape(2);
        nb.reqs.assign(B, ft_request{});
        nb.F.assign(B, 0);
        nb.T.assign(B, (uint32_t)T);
        nb.K = (uint32_t)K;
        for (size_t b = 0; b < B; ++b) {
          ft_request& q = nb.reqs[b];
          q.beams = beams.data() + b * T;
          q.num_beams = (uint32_t)T;
          q.num_steps = (uint32_t)T;
          q.topk = (uint32_t)K;
          q.topk_id = ids.data() + b * T * K;
          q.topk_logp = logp.data() + b * T * K;
          q.token_logp_threshold = token_logp_threshold;
          q.sent_logp_threshold = sent_logp_threshold;
          q.length_norm = length_norm;
          q.early_exit = early_exit;
          nb.F[b] = T ? q.beams[T - 1] : 0;
        }
        check_ft(ft_stage(c, nb.reqs.data(), B), "stage");
      },
      py::arg("trie"), py::arg("beams"), py::arg("topk_id"), py::arg("topk_logp"),
      py::arg("token_logp_threshold"), py::arg("sents_logp_threshold"),
      py::arg("length_norm"), py::arg("early_exit"));
  m.def(
      "launch",
      [](Trie& trie, size_t first, size_t count) {
        ft_ctx* c = ctx_of(trie);
        if (count == 0) check_ft(ft_launch(c), "launch");
        else check_ft(ft_launch_range(c, first, count), "launch");
      },
      py::arg("trie"), py::arg("first") = 0, py::arg("count") = 0);
  m.def(
      "reserve_staging",
      [](Trie& trie, size_t n) { check_ft(ft_reserve_staging(ctx_of(trie), n), "reserve_staging"); },
      py::arg("trie"), py::arg("max_staged"));
  m.def(
      "launch_times",
      [](Trie& trie, size_t n) {
        py::array_t<double> ms((py::ssize_t)n);
        int rc;
        {
          py::gil_scoped_release nogil;
          rc = ft_launch_times(ctx_of(trie), ms.mutable_data(), n);
        }
        check_ft(rc, "launch_times");
        return ms;
      },
      py::arg("trie"), py::arg("n"));
  m.def("sync", [](Trie& trie) {
    double ms = 0.0;
    {
      py::gil_scoped_release nogil;
      check_ft(ft_sync(ctx_of(trie), &ms), "sync");
    }
    return ms;
  });
  m.def("fetch", [](Trie& trie) {
    // returns (count[B], norms[B][F], lengths[B][F], tokens[B][F][T], timing)
    ft_ctx* c = ctx_of(trie);
    NpBatch& nb = staged_batch();
    const size_t B = nb.reqs.size();
    uint32_t Fm = 1, Tm = 1;
    for (size_t b = 0; b < B; ++b) {
      Fm = std::max(Fm, nb.F[b]);
      Tm = std::max(Tm, nb.T[b]);
    }
    py::array_t<uint32_t> count((py::ssize_t)B);
    py::array_t<double> norms({(py::ssize_t)B, (py::ssize_t)Fm});
    py::array_t<uint32_t> lens({(py::ssize_t)B, (py::ssize_t)Fm});
    py::array_t<uint32_t> toks({(py::ssize_t)B, (py::ssize_t)Fm, (py::ssize_t)Tm});
    py::array_t<double> dev({(py::ssize_t)B, (py::ssize_t)4});
    py::array_t<uint64_t> steps({(py::ssize_t)B, (py::ssize_t)Tm, (py::ssize_t)ftk_step_stats});
    std::memset(steps.mutable_data(), 0, B * Tm * ftk_step_stats * 8);
    std::memset(norms.mutable_data(), 0, B * Fm * 8);
    std::memset(lens.mutable_data(), 0, B * Fm * 4);
    std::memset(toks.mutable_data(), 0, B * Fm * Tm * 4);
    std::vector<ft_result> res(B);
    for (size_t b = 0; b < B; ++b) {
      std::memset(&res[b], 0, sizeof(ft_result));
      res[b].capacity = Fm;
      res[b].token_stride = Tm;
      res[b].logp_norm = norms.mutable_data() + b * Fm;
      res[b].length = lens.mutable_data() + b * Fm;
      res[b].tokens = toks.mutable_data() + b * Fm * Tm;
      res[b].step_stats = steps.mutable_data() + b * Tm * ftk_step_stats;
    }
    ft_timing tm{};
    int rc;
    {
      py::gil_scoped_release nogil;
      rc = ft_fetch(c, res.data(), B, &tm);
    }
    check_ft(rc, "fetch");
    for (size_t b = 0; b < B; ++b) {
      count.mutable_data()[b] = res[b].count;
      for (int i = 0; i < 4; ++i) dev.mutable_data()[b * 4 + i] = res[b].device_ms[i];
    }
    py::dict d;
    d["kernel_ms"] = tm.kernel_ms;
    d["expand_ms"] = tm.expand_ms;
    d["select_ms"] = tm.select_ms;
    d["other_ms"] = tm.other_ms;
    d["candidates"] = tm.candidates;
    d["parents"] = tm.parents;
    d["children"] = tm.children;
    d["probes"] = tm.probes;
    d["device_ms"] = dev;
    d["step_stats"] = steps;
    return py::make_tuple(count, norms, lens, toks, d);
  });

  // ---- synthetic generators ----------------------------------------------------
  m.def(
      "synth_keys",
      [](uint64_t n, uint32_t vocab, uint32_t lmin, uint32_t lmax, double s, uint64_t seed) {
        std::vector<uint32_t> toks;
        std::vector<uint64_t> offs;
        {
          py::gil_scoped_release nogil;
          ftamd::synth::make_keys(n, vocab, lmin, lmax, s, seed, &toks, &offs);
        }
        py::array_t<uint32_t> t((py::ssize_t)toks.size());
        py::array_t<uint64_t> o((py::ssize_t)offs.size());
        if (!toks.empty()) std::memcpy(t.mutable_data(), toks.data(), toks.size() * 4);
        std::memcpy(o.mutable_data(), offs.data(), offs.size() * 8);
        return py::make_tuple(t, o);
      },
      py::arg("n"), py::arg("vocab"), py::arg("lmin"), py::arg("lmax"), py::arg("s"),
      py::arg("seed"));
  m.def(
      "synth_paper_trie",
      [](Trie& trie, uint64_t n_keys, uint32_t vocab, double s, uint64_t seed,
         uint32_t lmin, uint32_t lmax, double p_end, int threads, uint64_t unique_keys) {
        // n_keys independent draws; with unique_keys > 0 the trie is then
        // topped up to exactly that many unique keys (prefix keys of length
        // >= lmin, see add_prefix_keys)
        ftamd::ImageBlob img;
        std::string err;
        bool ok;
        {
          py::gil_scoped_release nogil;
          ok = ftamd::synth::make_paper_trie(n_keys, vocab, s, lmin, lmax, p_end,
                                             seed, threads, &img, &err);
          if (ok && unique_keys)
            ok = ftamd::synth::add_prefix_keys(&img, unique_keys, lmin, seed, threads, &err);
        }
        if (!ok) throw marisa::Exception(MARISA_SIZE_ERROR, "synth_paper_trie: " + err);
        marisa::TrieImpl* im = trie.impl();
        im->drop_gpu();
        im->img.swap(img);
      },
      py::arg("trie"), py::arg("n_keys"), py::arg("vocab"), py::arg("s"),
      py::arg("seed"), py::arg("lmin") = 3, py::arg("lmax") = 16,
      py::arg("p_end") = 0.25, py::arg("threads") = 0, py::arg("unique_keys") = 0);
  // every key of a trie as (tokens, offsets), in lexicographic order (or,
  // with a nonzero seed, in a seeded random order): a depth-first walk of
  // the image (children in ascending first-token order), each node's edge
  // from first_tok or tail[]
  m.def(
      "keys_of",
      [](const Trie& trie, uint64_t shuffle_seed, bool progress) {
        auto say = [&](const char* what) {
          if (progress) {
            std::fprintf(stderr, "[keys_of] %s\n", what);
            std::fflush(stderr);
          }
        };
        const ftamd::ImageBlob& img = image_of(trie);
        const ft_node_rec* R = img.recs();
        const uint32_t* tail = img.tail();
        const uint64_t N = img.header().num_nodes;
        uint64_t nk = 0, nt = 0;
        for (uint64_t n = 0; n < N; ++n)
          if (R[n].meta & FT_META_TERMINAL) {
            ++nk;
            nt += R[n].meta & FT_META_DEPTH_MASK;
          }
        py::array_t<uint32_t> toks((py::ssize_t)nt);
        py::array_t<uint64_t> offs((py::ssize_t)(nk + 1));
        uint32_t* T = toks.mutable_data();
        uint64_t* O = offs.mutable_data();
        {
          py::gil_scoped_release nogil;
          // visit(f): f(key index in walk order, its tokens, length)
          auto walk = [&](auto&& f) {
            std::vector<uint32_t> pre, stack{0u};
            uint64_t k = 0;
            while (!stack.empty()) {
              const uint32_t n = stack.back();
              stack.pop_back();
              const uint32_t meta = R[n].meta;
              const uint32_t sd = meta & FT_META_DEPTH_MASK;
              const uint32_t el = (meta >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
              if (n != 0) {
                pre.resize(sd - el);
                for (uint32_t i = 0; i < el; ++i)
                  pre.push_back((meta & FT_META_LINK) ? tail[(uint64_t)R[n].tail_off + i]
                                                      : R[n].first_tok);
              }
              if (meta & FT_META_TERMINAL) f(k++, pre.data(), sd);
              for (uint32_t c = R[n + 1].child_begin; c > R[n].child_begin; --c)
                stack.push_back(c - 1);
            }
          };
          if (shuffle_seed == 0) {
            uint64_t o = 0;
            O[0] = 0;
            walk([&](uint64_t k, const uint32_t* p, uint32_t len) {
              std::memcpy(T + o, p, (size_t)len * 4);
              o += len;
              O[k + 1] = o;
            });
          } else {
            // slot[k]: where walk key k goes (a seeded Fisher-Yates
            // permutation); lengths in slot order, then their prefix
            std::vector<uint64_t> slot(nk);
            for (uint64_t k = 0; k < nk; ++k) slot[k] = k;
            uint64_t x = shuffle_seed * 0x9E3779B97F4A7C15ull + 1;
            for (uint64_t k = nk; k > 1; --k) {
              x ^= x >> 12;
              x ^= x << 25;
              x ^= x >> 27;
              const uint64_t r = (x * 0x2545F4914F6CDD1Dull) % k;
              std::swap(slot[k - 1], slot[r]);
            }
            say("order drawn");
            O[0] = 0;
            walk([&](uint64_t k, const uint32_t*, uint32_t len) { O[slot[k] + 1] = len; });
            for (uint64_t k = 0; k < nk; ++k) O[k + 1] += O[k];
            say("offsets placed");
            walk([&](uint64_t k, const uint32_t* p, uint32_t len) {
              std::memcpy(T + O[slot[k]], p, (size_t)len * 4);
            });
          }
          say("keys written");
        }
        return py::make_tuple(toks, offs);
      },
      py::arg("trie"), py::arg("shuffle_seed") = 0, py::arg("progress") = false);
  m.def(
      "validate_image",
      [](const Trie& trie) {
        std::string err;
        bool ok;
        {
          py::gil_scoped_release nogil;
          ok = ftamd::validate_image(image_of(trie), &err);
        }
        if (!ok) throw marisa::Exception(MARISA_FORMAT_ERROR, "validate_image: " + err);
      },
      py::arg("trie"));
  m.def(
      "synth_requests",
      [](const Trie& trie, uint64_t first, uint64_t count, uint32_t vocab, uint32_t steps,
         uint32_t topk, uint32_t seed_paths, double seed_mass, double sigma,
         bool analytic_rest, uint64_t seed, int threads, int model) {
        const ftamd::ImageBlob& img = image_of(trie);
        ftamd::synth::ProposalSpec sp;
        sp.vocab = vocab;
        sp.steps = steps;
        sp.topk = topk;
        sp.seed_paths = seed_paths;
        sp.seed_mass = seed_mass;
        sp.sigma = sigma;
        sp.analytic_rest = analytic_rest;
        sp.model = model == 1 ? ftamd::synth::ProposalSpec::kExample
                              : ftamd::synth::ProposalSpec::kSoftmax;
        py::array_t<uint32_t> ids({(py::ssize_t)count, (py::ssize_t)steps, (py::ssize_t)topk});
        py::array_t<float> lp({(py::ssize_t)count, (py::ssize_t)steps, (py::ssize_t)topk});
        uint32_t* ip = ids.mutable_data();
        float* fp = lp.mutable_data();
        {
          py::gil_scoped_release nogil;
          int nt = threads > 0 ? threads : (int)std::max(1u, std::thread::hardware_concurrency());
          nt = (int)std::min<uint64_t>((uint64_t)nt, std::max<uint64_t>(count, 1));
          std::atomic<uint64_t> nextr{0};
          std::vector<std::thread> pool;
          for (int w = 0; w < nt; ++w)
            pool.emplace_back([&]() {
              for (;;) {
                const uint64_t r = nextr.fetch_add(1);
                if (r >= count) break;
                ftamd::synth::make_request(img, sp, seed, first + r,
                                           ip + r * steps * topk, fp + r * steps * topk);
              }
            });
          for (auto& th : pool) th.join();
        }
        return py::make_tuple(ids, lp);
      },
      py::arg("trie"), py::arg("first"), py::arg("count"), py::arg("vocab"),
      py::arg("steps"), py::arg("topk"), py::arg("seed_paths"), py::arg("seed_mass"),
      py::arg("sigma"), py::arg("analytic_rest"), py::arg("seed"), py::arg("threads") = 0,
      py::arg("model") = 0);
}
