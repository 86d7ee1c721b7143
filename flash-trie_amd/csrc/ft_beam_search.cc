// ft_beam_search.cc -- the beam-search command line tool.
//
// Same usage, arguments and printed lines as the reference's
// marisa-beam-search (tools/marisa-beam-search.cc:151-343):
//
//   ft-beam-search [OPTION]... DATASET_DIR [BEAM_WIDTH [BATCH_SIZE]]
//
// loads DATASET_DIR/marisa_trie.bin (a MARISA trie file or a trie image),
// reads DATASET_DIR/topk_keys.txt and topk_scores.txt, and runs the first 100
// requests with thresholds -7 / -40 and length norm 5: the host search with
// per-request times, then with -g the GPU search in batches of BATCH_SIZE.
// TBS_TIMING_CSV=<path> writes one row per request with the device phase
// times.  -a compares the host and GPU results of every request: the same
// sequences in the same order with the same scores (the reference checks
// key ids found by lookup, to 1e-4); it also reports how many outputs are
// keys of the trie, as the reference does.
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <numeric>
#include <string>
#include <vector>

#include "../../include/flashtrie_amd.h"
#include "marisa.h"
#include "marisa/topk_io.h"
#include "trie_impl.h"

using namespace marisa;

namespace {

bool mmap_flag = false;
bool test_gpu = false;
bool check_accuracy = false;
bool early_exit = false;

void print_help(const char* cmd) {
  std::cerr << "Usage: " << cmd
            << " [OPTION]... DATASET_DIR [BEAM_WIDTH [BATCH_SIZE]]\n\n"
               "Options:\n"
               "  -m, --mmap-dictionary  use memory-mapped I/O to load a dictionary\n"
               "  -r, --read-dictionary  read an entire dictionary into memory"
               " (default)\n"
               "  -g, --test-gpu         test gpu beam search\n"
               "  -a, --check-accuracy   compare cpu and gpu beam search output\n"
               "  -e, --early-exit       early exit during beam search\n"
               "  -h, --help             print this help\n"
            << std::endl;
}

double msec(std::chrono::steady_clock::time_point a,
            std::chrono::steady_clock::time_point b) {
  return std::chrono::duration<double, std::milli>(b - a).count();
}

// Is `q` a key of the trie?  Walks the image from the root: binary search of
// each node's children by first token, then the rest of a link edge.
bool is_key(const ft_image_header* h, const std::vector<Label>& q) {
  const uint8_t* base = (const uint8_t*)h;
  const ft_node_rec* R = (const ft_node_rec*)(base + h->recs_offset);
  const uint32_t* TL = (const uint32_t*)(base + h->tail_offset);
  uint32_t v = 0;
  size_t i = 0;
  while (i < q.size()) {
    uint32_t lo = R[v].child_begin, hi = R[v + 1].child_begin;
    while (lo < hi) {
      const uint32_t mid = lo + (hi - lo) / 2;
      if (R[mid].first_tok < q[i]) lo = mid + 1; else hi = mid;
    }
    if (lo == R[v + 1].child_begin || R[lo].first_tok != q[i]) return false;
    const uint32_t m = R[lo].meta;
    const uint32_t el = (m >> FT_META_ELEN_SHIFT) & FT_META_ELEN_MASK;
    if (m & FT_META_LINK) {
      if (i + el > q.size()) return false;
      for (uint32_t j = 0; j < el; ++j)
        if (TL[R[lo].tail_off + j] != q[i + j]) return false;
    }
    i += el;
    v = lo;
  }
  return (R[v].meta & FT_META_TERMINAL) != 0;
}

size_t count_keys(const Trie& trie, const std::vector<std::vector<Label>>& sents) {
  const ft_image_header* h = (const ft_image_header*)trie.image_data();
  size_t n = 0;
  for (const auto& s : sents) n += is_key(h, s);
  return n;
}

bool same_results(const std::vector<std::vector<Label>>& a, const std::vector<double>& as,
                  const std::vector<std::vector<Label>>& b, const std::vector<double>& bs) {
  if (a.size() != b.size()) {
    std::printf("Mismatch in beam count, cpu %zu != gpu %zu\n", a.size(), b.size());
    return false;
  }
  for (size_t i = 0; i < a.size(); ++i) {
    if (a[i] != b[i]) {
      std::printf("Mismatch in beam %zu tokens\n", i);
      return false;
    }
    if (as[i] != bs[i]) {
      std::printf("Mismatch in beam %zu score cpu %.17g != gpu %.17g\n", i, as[i], bs[i]);
      return false;
    }
  }
  return true;
}

int beam_search(const std::vector<std::string>& args) {
  if (args.empty()) {
    std::cerr << "error: dictionary is not specified" << std::endl;
    return 10;
  } else if (args.size() > 3) {
    std::cerr << "more than 3 arguments are not allowed" << std::endl;
    return 11;
  }
  const std::string dataset_dir = args[0];
  const std::string trie_path = dataset_dir + "/marisa_trie.bin";
  std::cout << "Trie path " << trie_path << std::endl;
  Trie trie;
  try {
    if (mmap_flag) trie.mmap(trie_path.c_str()); else trie.load(trie_path.c_str());
  } catch (const Exception& ex) {
    std::cerr << ex.what() << ": failed to " << (mmap_flag ? "mmap" : "load")
              << " a dictionary file: " << dataset_dir << std::endl;
    return mmap_flag ? 20 : 21;
  }
  std::cout << "Finished loading trie" << std::endl;

  std::vector<std::vector<std::vector<Label>>> topk_ids;
  std::vector<std::vector<std::vector<float>>> topk_logps;
  try {
    std::tie(topk_ids, topk_logps) = load_topk_keys_and_scores(dataset_dir);
  } catch (const Exception& ex) {
    std::cerr << ex.what() << std::endl;
    return 30;
  }
  if (topk_ids.empty()) {
    std::cerr << "error: no requests in " << dataset_dir << std::endl;
    return 31;
  }
  const size_t num_requests = topk_ids.size();
  const size_t max_output_len = topk_ids[0].size();
  const float token_logp_threshold = -7.0f;
  const double sent_logp_threshold = -40.0;
  const double length_norm = 5;
  const UInt32 beam_width = args.size() >= 2 ? (UInt32)std::stoi(args[1]) : 200;
  const size_t batch_size = args.size() >= 3 ? (size_t)std::stoi(args[2]) : 1;
  std::vector<UInt32> beams(max_output_len, beam_width);
  if (test_gpu) {
    try {
      trie.init_tbs_gpu(batch_size);
    } catch (const Exception& ex) {
      std::cerr << ex.what() << std::endl;
      return 40;
    }
    int num_cus = 0;
    if (ft_device_info(trie.impl()->ctx, &num_cus, nullptr, nullptr, nullptr, 0) == FT_OK)
      std::cout << "GPU CUs " << num_cus << std::endl;
  }
  const size_t first_req = 0;
  const size_t last_req = std::min<size_t>(100 + first_req, num_requests);

  // host search, one request at a time
  std::vector<std::vector<std::vector<Label>>> cpu_sent(last_req);
  std::vector<std::vector<double>> cpu_norm(last_req);
  std::vector<double> times;
  for (size_t r = first_req; r < last_req; ++r) {
    TbsInput in{beams, topk_ids[r], topk_logps[r], cpu_sent[r], cpu_norm[r],
                token_logp_threshold, sent_logp_threshold, length_norm, early_exit};
    const auto a = std::chrono::high_resolution_clock::now();
    trie.tbs(in);
    const auto b = std::chrono::high_resolution_clock::now();
    times.push_back(get_msec(a, b));
    if (!check_accuracy)
      std::printf("Req #%zu: %zu beams generated in %.2f msec\n", r, cpu_sent[r].size(),
                  times.back());
  }
  std::printf("Measured time per request in CPU tbs: %.2f msec\n",
              std::accumulate(times.begin(), times.end(), 0.0) / (double)times.size());
  if (!test_gpu) return 0;

  std::ofstream timing_csv;
  if (const char* p = std::getenv("TBS_TIMING_CSV")) {
    timing_csv.open(p);
    timing_csv << "req_id,beam_width,batch_size,num_beams,kernel_ms,host_batch_ms,"
                  "t_expansion_ms,t_validation_ms,t_selection_ms,t_grid_overhead_ms\n";
    std::cout << "Writing per-request timing breakdown to " << p << std::endl;
  }
  std::vector<std::vector<std::vector<Label>>> gpu_sent(last_req);
  std::vector<std::vector<double>> gpu_norm(last_req);
  size_t num_batches = 0, mismatches = 0;
  const auto start = std::chrono::steady_clock::now();
  for (size_t r0 = first_req; r0 < last_req; r0 += batch_size, ++num_batches) {
    const size_t n = std::min(last_req - r0, batch_size);
    std::vector<TbsInput> inputs;
    std::printf("Reqs:");
    for (size_t i = 0; i < n; ++i) {
      std::printf(" %zu", r0 + i);
      inputs.push_back(TbsInput{beams, topk_ids[r0 + i], topk_logps[r0 + i], gpu_sent[r0 + i],
                                gpu_norm[r0 + i], token_logp_threshold, sent_logp_threshold,
                                length_norm, early_exit});
    }
    std::printf(" ");
    const auto a = std::chrono::steady_clock::now();
    try {
      trie.tbs_gpu_batched(inputs);
    } catch (const Exception& ex) {
      std::printf("\n");
      std::cerr << ex.what() << std::endl;
      return 41;
    }
    const double batch_ms = msec(a, std::chrono::steady_clock::now());
    std::printf("Beams:");
    for (size_t i = 0; i < n; ++i) std::printf(" %zu", gpu_sent[r0 + i].size());
    std::printf(" Time: %.2f msec\n", batch_ms);
    if (timing_csv.is_open())
      for (size_t i = 0; i < n; ++i) {
        const TbsInput& in = inputs[i];
        timing_csv << (r0 + i) << ',' << beam_width << ',' << n << ','
                   << gpu_sent[r0 + i].size() << ',' << in.kernel_ms << ',' << batch_ms
                   << ',' << in.t_expansion_ms << ',' << in.t_validation_ms << ','
                   << in.t_selection_ms << ',' << in.t_grid_overhead_ms << '\n';
      }
  }
  const double loop_ms = msec(start, std::chrono::steady_clock::now());
  if (check_accuracy) {
    for (size_t r = first_req; r < last_req; ++r) {
      std::cout << "Checking accuracy for req_id " << r << std::endl;
      std::cout << "CPU valid beams " << count_keys(trie, cpu_sent[r]) << "/"
                << cpu_sent[r].size() << std::endl;
      std::cout << "GPU valid beams " << count_keys(trie, gpu_sent[r]) << "/"
                << gpu_sent[r].size() << std::endl;
      if (!same_results(cpu_sent[r], cpu_norm[r], gpu_sent[r], gpu_norm[r])) {
        std::printf("Mismatch in req_id %zu\n", r);
        ++mismatches;
      }
    }
    std::printf("%zu/%zu requests identical on CPU and GPU\n",
                (last_req - first_req) - mismatches, last_req - first_req);
  }
  std::printf("Total time to process %zu requests with %zu batch size: %.2f msec\n",
              last_req - first_req, batch_size, loop_ms);
  std::printf("Per batch latency  : %.2f msec\n", loop_ms / (double)num_batches);
  std::printf("Per request latency: %.2f msec\n", loop_ms / (double)(last_req - first_req));
  return mismatches ? 50 : 0;
}

}  // namespace

int main(int argc, char* argv[]) {
  std::vector<std::string> args;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "-m" || a == "--mmap-dictionary") {
      mmap_flag = true;
    } else if (a == "-r" || a == "--read-dictionary") {
      mmap_flag = false;
    } else if (a == "-g" || a == "--test-gpu") {
      test_gpu = true;
    } else if (a == "-a" || a == "--check-accuracy") {
      check_accuracy = true;
    } else if (a == "-e" || a == "--early-exit") {
      early_exit = true;
    } else if (a == "-h" || a == "--help") {
      print_help(argv[0]);
      return 0;
    } else if (a.size() > 1 && a[0] == '-') {
      std::cerr << "error: unknown option " << a << std::endl;
      print_help(argv[0]);
      return 1;
    } else {
      args.push_back(a);
    }
  }
  return beam_search(args);
}
