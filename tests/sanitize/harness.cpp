// Host harness for the sanitizer build (tests/test_sanitize.py): drives the
// product's host-only C ABI code (tiga-lang_amd/csrc/tgx_capi.cpp: status
// strings, error messages, the reference planner restatement) and the C CPU
// baseline (oracle/cpu_native.c) from a line protocol on stdin, printing the
// results for the test to compare with the Python oracle.
//
//   plan <rows> <max> <sum> <has_node> <n_hist> <hist...>
//     -> plan <code> <util> <n> <bounds...> <mapping...> <rows_in...> <ppr> <active>
//   sum <n_dst> <n_src> <F> <threads> <row_ptr...> <col...> <x...> <w...> <dout...>
//     -> sum <out...> | <dx...> | <dw...>
//   bad
//     -> bad <status> <message>   (a planner call with a null output)
#include <cstdint>
#include <cstdio>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "tgx.h"

extern "C" int tgx_oracle_csr_sum_fwd(const int64_t* row_ptr, const int64_t* col, const float* x,
                                      const float* w, float* out, int64_t n_dst, int64_t F,
                                      int threads);
extern "C" int tgx_oracle_csr_sum_bwd_lowered(const int64_t* row_ptr, const int64_t* col,
                                              const float* x, const float* w, const float* dout,
                                              float* dx, float* dw, float* dmsg_scratch,
                                              int64_t n_dst, int64_t n_src, int64_t F);

template <typename T>
static std::vector<T> read_n(std::istringstream& in, int64_t n) {
  std::vector<T> v(static_cast<size_t>(n));
  for (auto& x : v) in >> x;
  return v;
}

int main() {
  std::string line;
  while (std::getline(std::cin, line)) {
    std::istringstream in(line);
    std::string op;
    in >> op;
    if (op == "plan") {
      int64_t rows, max_deg, sum, n_hist;
      int has_node;
      in >> rows >> max_deg >> sum >> has_node >> n_hist;
      std::vector<int64_t> hist = read_n<int64_t>(in, n_hist);
      int code = -1, n = 0, mapping[64];
      int64_t util = 0, bounds[64], rows_in[64], ppr = 0, active = 0;
      const int st = tgx_plan_reference_buckets(rows, max_deg, sum, n_hist ? hist.data() : nullptr,
                                                has_node, &code, &util, bounds, mapping, rows_in,
                                                &n, &ppr, &active);
      if (st != TGX_OK) {
        std::printf("error %d %s\n", st, tgx_last_error());
        continue;
      }
      std::printf("plan %d %lld %d", code, static_cast<long long>(util), n);
      for (int k = 0; k < n; ++k) std::printf(" %lld", static_cast<long long>(bounds[k]));
      for (int k = 0; k < n; ++k) std::printf(" %d", mapping[k]);
      for (int k = 0; k < n; ++k) std::printf(" %lld", static_cast<long long>(rows_in[k]));
      std::printf(" %lld %lld\n", static_cast<long long>(ppr), static_cast<long long>(active));
    } else if (op == "sum") {
      int64_t n_dst, n_src, F;
      int threads;
      in >> n_dst >> n_src >> F >> threads;
      std::vector<int64_t> rp = read_n<int64_t>(in, n_dst + 1);
      const int64_t E = rp.back();
      std::vector<int64_t> col = read_n<int64_t>(in, E);
      std::vector<float> x = read_n<float>(in, n_src * F), w = read_n<float>(in, E);
      std::vector<float> dout = read_n<float>(in, n_dst * F);
      std::vector<float> out(n_dst * F), dx(n_src * F), dw(E), scratch(E * F + 1);
      if (tgx_oracle_csr_sum_fwd(rp.data(), col.data(), x.data(), w.data(), out.data(), n_dst,
                                 F, threads) != 0 ||
          tgx_oracle_csr_sum_bwd_lowered(rp.data(), col.data(), x.data(), w.data(), dout.data(),
                                         dx.data(), dw.data(), scratch.data(), n_dst, n_src,
                                         F) != 0) {
        std::printf("error\n");
        continue;
      }
      std::printf("sum");
      for (float v : out) std::printf(" %.9g", v);
      std::printf(" |");
      for (float v : dx) std::printf(" %.9g", v);
      std::printf(" |");
      for (float v : dw) std::printf(" %.9g", v);
      std::printf("\n");
    } else if (op == "bad") {
      const int st = tgx_plan_reference_buckets(4, 8, 16, nullptr, 0, nullptr, nullptr, nullptr,
                                                nullptr, nullptr, nullptr, nullptr, nullptr);
      std::printf("bad %d %s %s\n", st, tgx_status_string(st), tgx_last_error());
    }
    std::fflush(stdout);
  }
  return 0;
}
