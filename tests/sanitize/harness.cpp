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
//   twins <seed> <n> <H> <D>
//     -> twins ok | twins fail <what>
//        every CPU twin (tiga-lang_amd/csrc/tgx_cpu.cpp) on a random graph with
//        hub rows above the 512-edge wave bound (split into chunks), run at 1
//        and 4 threads with the results compared bit for bit, then the
//        argument checks on broken inputs (a column out of range, a plan
//        listing a row twice, a perm that is no permutation).
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <iostream>
#include <random>
#include <sstream>
#include <string>
#include <vector>

#include "tgx.h"
#include "tgx_cpu.h"

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

namespace {

struct Plan {
  std::vector<int32_t> rows, chunks;
  tgx_row_plan p{};
};

bool make_plan(const void* rp, int bits, int64_t n, Plan* out) {
  out->rows.assign(static_cast<size_t>(n > 0 ? n : 1), 0);
  const int64_t bounds[3] = {0, 512, int64_t{1} << 62};
  int64_t off[4];
  if (tgx_cpu_plan_degree_bins(rp, bits, n, bounds, 3, out->rows.data(), off) != TGX_OK)
    return false;
  const int64_t n_split = off[3] - off[2];
  out->chunks.assign(static_cast<size_t>(n_split + 1), 0);
  int64_t n_chunks = 0;
  if (tgx_cpu_plan_split_chunks(rp, bits, out->rows.data() + off[2], n_split, 512,
                                out->chunks.data(), &n_chunks) != TGX_OK)
    return false;
  out->p = tgx_row_plan{n, off[1] - off[0], off[2] - off[1], n_split, n_chunks, 512, 512,
                        out->rows.data(), out->chunks.data()};
  return true;
}

template <typename T>
bool same(const std::vector<T>& a, const std::vector<T>& b) {
  return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(T)) == 0;
}

// Returns "" when every twin ran and agreed across thread counts, else what failed.
std::string run_twins(uint64_t seed, int64_t n, int H, int D) {
  std::mt19937_64 rng(seed);
  std::normal_distribution<float> normal(0.f, 1.f);
  std::vector<int64_t> rp(static_cast<size_t>(n) + 1, 0);
  for (int64_t i = 0; i < n; ++i) {
    int64_t deg = static_cast<int64_t>(rng() % 9);
    if (i % 97 == 5) deg = 513 + static_cast<int64_t>(rng() % 900);
    if (i % 11 == 3) deg = 0;
    rp[i + 1] = rp[i] + deg;
  }
  const int64_t E = rp[n];
  std::vector<int64_t> col(static_cast<size_t>(E));
  for (auto& c : col) c = static_cast<int64_t>(rng() % static_cast<uint64_t>(n));
  std::vector<int32_t> rpt(n + 1), colt(E), perm(E), inv(E);
  if (tgx_cpu_csr_transpose(rp.data(), col.data(), 64, n, n, E, rpt.data(), colt.data(),
                            perm.data(), inv.data()) != TGX_OK)
    return "transpose";
  std::vector<int32_t> dst(E);
  if (tgx_cpu_destination_index(rp.data(), 64, n, E, dst.data(), 32) != TGX_OK)
    return "destination_index";
  Plan plan, plan_t;
  if (!make_plan(rp.data(), 64, n, &plan) || !make_plan(rpt.data(), 32, n, &plan_t))
    return "plan";
  if (plan.p.n_split == 0) return "no split rows";
  auto fill = [&](int64_t count) {
    std::vector<float> v(static_cast<size_t>(count));
    for (auto& x : v) x = normal(rng);
    return v;
  };
  auto bf16 = [&](int64_t count) {  // bf16 bit patterns of normal samples
    std::vector<uint16_t> v(static_cast<size_t>(count));
    for (auto& x : v) {
      float f = normal(rng);
      uint32_t u;
      std::memcpy(&u, &f, 4);
      x = static_cast<uint16_t>(u >> 16);
    }
    return v;
  };
  const int64_t F = 5, HD = static_cast<int64_t>(H) * D;
  const std::vector<float> x = fill(n * F), w = fill(E), g = fill(n * F);
  const std::vector<float> h = fill(n * HD), a = fill(2 * HD), dh_in = fill(n * HD);
  const std::vector<uint16_t> q = bf16(n * HD), k = bf16(n * HD), v = bf16(n * HD),
                              go = bf16(n * HD);
  const std::vector<float> bias = fill(E * H);
  std::vector<float> sums[2], gats[2];
  std::vector<uint16_t> dots[2];
  for (int r = 0; r < 2; ++r) {
    tgx_cpu_set_threads(r == 0 ? 1 : 4);
    std::vector<float> out(n * F), dx(n * F), dw(E);
    if (tgx_cpu_csr_sum_fwd(rp.data(), col.data(), 64, &plan.p, x.data(), w.data(), out.data(),
                            n, n, F, TGX_DTYPE_F32) != TGX_OK ||
        tgx_cpu_csr_sum_bwd(rpt.data(), colt.data(), perm.data(), &plan_t.p, x.data(), w.data(),
                            g.data(), dx.data(), dw.data(), n, n, F, TGX_DTYPE_F32) != TGX_OK)
      return "sum";
    sums[r] = out;
    sums[r].insert(sums[r].end(), dx.begin(), dx.end());
    sums[r].insert(sums[r].end(), dw.begin(), dw.end());
    std::vector<float> ho(n * HD), ns(n * H * 4), dh(n * HD), das(HD), dad(HD);
    if (tgx_cpu_gat_fwd(rp.data(), col.data(), 64, &plan.p, h.data(), h.data(), a.data(),
                        a.data() + HD, 0.2f, ho.data(), ns.data(), n, n, H, D,
                        TGX_DTYPE_F32) != TGX_OK ||
        tgx_cpu_gat_bwd(rp.data(), col.data(), 64, &plan.p, rpt.data(), colt.data(), perm.data(),
                        inv.data(), &plan_t.p, h.data(), h.data(), a.data(), a.data() + HD, 0.2f,
                        ho.data(), ns.data(), dh_in.data(), dh.data(), dh.data(), das.data(),
                        dad.data(), n, n, E, H, D, TGX_DTYPE_F32) != TGX_OK)
      return std::string("gat: ") + tgx_last_error();
    gats[r] = ho;
    gats[r].insert(gats[r].end(), dh.begin(), dh.end());
    gats[r].insert(gats[r].end(), das.begin(), das.end());
    gats[r].insert(gats[r].end(), dad.begin(), dad.end());
    std::vector<uint16_t> o(n * HD), dq(n * HD), dk(n * HD), dv(n * HD);
    std::vector<float> ml(n * H * 2), db(E * H);
    if (D % 8 == 0) {
      if (tgx_cpu_dot_attn_fwd(rp.data(), col.data(), 64, &plan.p, q.data(), k.data(), v.data(),
                               bias.data(), 0.125f, o.data(), ml.data(), n, n, H, D,
                               TGX_DTYPE_BF16) != TGX_OK ||
          tgx_cpu_dot_attn_bwd(rp.data(), col.data(), 64, &plan.p, rpt.data(), colt.data(),
                               perm.data(), &plan_t.p, q.data(), k.data(), v.data(), bias.data(),
                               0.125f, o.data(), ml.data(), go.data(), dq.data(), dk.data(),
                               dv.data(), db.data(), n, n, H, D, TGX_DTYPE_BF16) != TGX_OK)
        return std::string("dot: ") + tgx_last_error();
    }
    dots[r] = o;
    dots[r].insert(dots[r].end(), dq.begin(), dq.end());
    dots[r].insert(dots[r].end(), dk.begin(), dk.end());
    dots[r].insert(dots[r].end(), dv.begin(), dv.end());
    if (D == 64 || D == 128) {
      const int32_t cu[4] = {0, static_cast<int32_t>(n / 3), static_cast<int32_t>(n / 3),
                             static_cast<int32_t>(n)};
      const int64_t strides[4] = {HD, D, HD, D};
      std::vector<uint16_t> ao(n * HD), aq(n * HD), ak(n * HD), av(n * HD);
      std::vector<float> lse(n * H), delta(n * H);
      if (tgx_cpu_attn_fwd(cu, cu, 3, 1, TGX_DTYPE_F16, q.data(), k.data(), v.data(), strides,
                           0.125f, 0.f, ao.data(), lse.data(), n, n, H, D) != TGX_OK ||
          tgx_cpu_attn_bwd(cu, cu, 3, 1, TGX_DTYPE_F16, q.data(), k.data(), v.data(), strides,
                           ao.data(), lse.data(), go.data(), 0.125f, aq.data(), ak.data(),
                           av.data(), delta.data(), n, n, H, D) != TGX_OK)
        return std::string("attn: ") + tgx_last_error();
      dots[r].insert(dots[r].end(), aq.begin(), aq.end());
    }
  }
  tgx_cpu_set_threads(0);
  if (!same(sums[0], sums[1])) return "sum differs across thread counts";
  if (!same(gats[0], gats[1])) return "gat differs across thread counts";
  if (!same(dots[0], dots[1])) return "attention differs across thread counts";
  // Broken inputs are rejected, not read out of bounds.
  std::vector<float> out(n * F);
  std::vector<int64_t> bad_col = col;
  bad_col[E / 2] = n + 7;
  if (tgx_cpu_csr_sum_fwd(rp.data(), bad_col.data(), 64, &plan.p, x.data(), w.data(),
                          out.data(), n, n, F, TGX_DTYPE_F32) != TGX_INVALID_ARGUMENT)
    return "column out of range accepted";
  Plan twice = plan;
  twice.rows[1] = twice.rows[0];
  twice.p.rows_dev = twice.rows.data();
  twice.p.chunk_offsets_dev = twice.chunks.data();
  if (tgx_cpu_csr_sum_fwd(rp.data(), col.data(), 64, &twice.p, x.data(), w.data(), out.data(),
                          n, n, F, TGX_DTYPE_F32) != TGX_INVALID_ARGUMENT)
    return "plan with a repeated row accepted";
  std::vector<int32_t> bad_perm = perm;
  bad_perm[0] = bad_perm[1];
  std::vector<float> dx(n * F);
  if (tgx_cpu_csr_sum_bwd(rpt.data(), colt.data(), bad_perm.data(), &plan_t.p, x.data(),
                          w.data(), g.data(), dx.data(), nullptr, n, n, F, TGX_DTYPE_F32) !=
      TGX_INVALID_ARGUMENT)
    return "broken perm accepted";
  return "";
}

}  // namespace

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
    } else if (op == "twins") {
      uint64_t seed;
      int64_t n;
      int H, D;
      in >> seed >> n >> H >> D;
      const std::string fail = run_twins(seed, n, H, D);
      if (fail.empty())
        std::printf("twins ok\n");
      else
        std::printf("twins fail %s\n", fail.c_str());
    } else if (op == "bad") {
      const int st = tgx_plan_reference_buckets(4, 8, 16, nullptr, 0, nullptr, nullptr, nullptr,
                                                nullptr, nullptr, nullptr, nullptr, nullptr);
      std::printf("bad %d %s %s\n", st, tgx_status_string(st), tgx_last_error());
    }
    std::fflush(stdout);
  }
  return 0;
}
