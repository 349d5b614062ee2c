// nova-run: run a Nova program (op-surface .mlir text) through libnova_run.
//
//   nova-run FILE.mlir [--func NAME] [--plan] [--seed N] [--reps K]
//
// --plan prints each function's launch plan (no GPU needed).  Otherwise the
// function's arguments are filled from a counter-based generator
// (splitmix64 of seed and element index: floats uniform in [-1, 1) rounded
// to the argument's dtype, integer arguments (i16 / i32 / i64) uniform in
// [0, C) with C the smallest dim of the rank-2 float arguments, at most
// 65536), the function runs --reps times,
// and each result's sum and max |x| are printed with the time per run
// (host<->device copies included).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <cmath>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/nova_run.h"

namespace {
uint64_t splitmix(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
uint16_t to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
float from_bits(int dt, const void *p, int64_t i) {
  if (dt == 0) return ((const float *)p)[i];
  if (dt == 1) {
    uint32_t u = (uint32_t)((const uint16_t *)p)[i] << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
  }
  if (dt == 2) return (float)((const _Float16 *)p)[i];
  if (dt == 3) return (float)((const int32_t *)p)[i];
  if (dt == 5) return (float)((const uint16_t *)p)[i];
  return (float)((const int64_t *)p)[i];
}
// dtype codes: 0 f32, 1 bf16, 2 f16, 3 i32, 4 i64, 5 i16
int esize(int dt) { return dt == 0 || dt == 3 ? 4 : dt == 4 ? 8 : 2; }
}  // namespace

int main(int argc, char **argv) {
  const char *file = nullptr, *func = nullptr;
  bool plan_only = false;
  uint64_t seed = 0;
  int reps = 1;
  for (int i = 1; i < argc; ++i) {
    if (!strcmp(argv[i], "--func") && i + 1 < argc) func = argv[++i];
    else if (!strcmp(argv[i], "--plan")) plan_only = true;
    else if (!strcmp(argv[i], "--seed") && i + 1 < argc) seed = strtoull(argv[++i], nullptr, 10);
    else if (!strcmp(argv[i], "--reps") && i + 1 < argc) reps = atoi(argv[++i]);
    else if (argv[i][0] != '-') file = argv[i];
    else {
      fprintf(stderr, "usage: nova-run FILE.mlir [--func NAME] [--plan] [--seed N] [--reps K]\n");
      return 2;
    }
  }
  if (!file) {
    fprintf(stderr, "usage: nova-run FILE.mlir [--func NAME] [--plan] [--seed N] [--reps K]\n");
    return 2;
  }
  std::ifstream in(file);
  if (!in) {
    fprintf(stderr, "nova-run: cannot read %s\n", file);
    return 2;
  }
  std::stringstream ss;
  ss << in.rdbuf();
  NovaRunProgram *p = nova_run_parse(ss.str().c_str());
  if (!p) {
    fprintf(stderr, "nova-run: %s\n", nova_run_last_error());
    return 1;
  }
  int rc = 0;
  for (int f = 0; f < nova_run_num_funcs(p); ++f) {
    const char *name = nova_run_func_name(p, f);
    if (func && strcmp(func, name)) continue;
    std::vector<char> text(1 << 16);
    if (nova_run_plan(p, name, text.data(), text.size())) {
      fprintf(stderr, "nova-run: @%s: %s\n", name, nova_run_last_error());
      rc = 1;
      continue;
    }
    printf("%s", text.data());
    if (plan_only) continue;
    const int na = nova_run_num_args(p, name), nr = nova_run_num_results(p, name);
    std::vector<std::vector<char>> args(na), res(nr);
    std::vector<const void *> pa(na);
    std::vector<void *> pr(nr);
    // Integer arguments (labels, gather / scatter indices) stay below the
    // smallest dim of every rank-2 float argument, so they are in range for
    // any table or class dimension of the program.
    int64_t classes = 65536;
    for (int a = 0; a < na; ++a) {
      int32_t dt, rank;
      int64_t shape[8];
      nova_run_arg_info(p, name, a, &dt, &rank, shape);
      if (rank == 2 && dt <= 2)
        for (int d = 0; d < 2; ++d)
          if (shape[d] > 0 && shape[d] < classes) classes = shape[d];
    }
    for (int a = 0; a < na; ++a) {
      int32_t dt, rank;
      int64_t shape[8], n = 1;
      nova_run_arg_info(p, name, a, &dt, &rank, shape);
      for (int d = 0; d < rank; ++d) n *= shape[d];
      args[a].resize((size_t)n * esize(dt));
      for (int64_t i = 0; i < n; ++i) {
        const uint64_t r = splitmix(seed * 0x100000001ull + (uint64_t)a * 0x1000000000ull + (uint64_t)i);
        const float u = (float)((r >> 40) * (1.0 / 16777216.0)) * 2.0f - 1.0f;
        if (dt == 0) ((float *)args[a].data())[i] = u;
        else if (dt == 1) ((uint16_t *)args[a].data())[i] = to_bf16(u);
        else if (dt == 2) ((_Float16 *)args[a].data())[i] = (_Float16)u;
        else if (dt == 3) ((int32_t *)args[a].data())[i] = (int32_t)(r % (uint64_t)classes);
        else if (dt == 5) ((uint16_t *)args[a].data())[i] = (uint16_t)(r % (uint64_t)classes);
        else ((int64_t *)args[a].data())[i] = (int64_t)(r % (uint64_t)classes);
      }
      pa[a] = args[a].data();
    }
    for (int r = 0; r < nr; ++r) {
      int32_t dt, rank;
      int64_t shape[8], n = 1;
      nova_run_result_info(p, name, r, &dt, &rank, shape);
      for (int d = 0; d < rank; ++d) n *= shape[d];
      res[r].resize((size_t)n * esize(dt));
      pr[r] = res[r].data();
    }
    const auto t0 = std::chrono::steady_clock::now();
    for (int k = 0; k < reps && !rc; ++k)
      if (nova_run_execute(p, name, pa.data(), pr.data())) {
        fprintf(stderr, "nova-run: @%s: %s\n", name, nova_run_last_error());
        rc = 1;
      }
    const double ms =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() /
        reps;
    if (rc) continue;
    for (int r = 0; r < nr; ++r) {
      int32_t dt, rank;
      int64_t shape[8], n = 1;
      nova_run_result_info(p, name, r, &dt, &rank, shape);
      for (int d = 0; d < rank; ++d) n *= shape[d];
      double sum = 0, mx = 0;
      for (int64_t i = 0; i < n; ++i) {
        const double v = from_bits(dt, res[r].data(), i);
        sum += v;
        mx = std::fmax(mx, std::fabs(v));
      }
      printf("  result %d: %lld elements, sum %.6g, max|x| %.6g\n", r, (long long)n, sum, mx);
    }
    printf("  %.3f ms per run (copies included)\n", ms);
  }
  nova_run_free(p);
  return rc;
}
