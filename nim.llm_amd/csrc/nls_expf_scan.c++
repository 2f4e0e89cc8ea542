// nls_expf_scan -- exhaustive check of nls::expf_cr and nls::expf_cr_t over
// every binary32 input whose exponential is finite and non-zero, against
// (float)expl(x) (64-bit significand).  Build-time tool: writes
// nls_expf_table.h (the inputs where either float64 evaluation cannot decide
// the rounding, with their correctly rounded results) and prints a summary.
// Inputs where expl itself lies within 2^-60 of a rounding boundary are
// printed for a high-precision check.
//
//   g++ -O2 -ffp-contract=off -pthread nls_expf_scan.c++ -o scan
//   ./scan table    -> rewrites nls_expf_table.h
//   ./scan verify   -> checks expf_cr and expf_cr_t == (float)expl everywhere;
//                      prints a checksum of each (they must agree)
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "nls_expf.h"

static const uint32_t kNegEnd = 0xC2D00000u;  // -104.0f
static const uint32_t kPosEnd = 0x42B20000u;  // 89.0f

struct Job {
  uint64_t lo, hi;  // index range over the combined domain
  int mode;
  std::vector<uint32_t> hard_in, hard_out, amb;
  uint64_t mismatches = 0;
  double max_rel = 0, max_rel_t = 0;
  uint64_t checksum = 0, checksum_t = 0;
  uint64_t count = 0;
};

static inline uint32_t index_to_bits(uint64_t i) {
  const uint64_t nneg = kNegEnd - 0x80000000u;
  if (i < nneg) return 0x80000000u + (uint32_t)i;  // -0 .. just above -104
  return (uint32_t)(i - nneg);                     // +0 .. just below 89
}

static inline uint64_t mix(uint64_t z) {
  z += 0x9e3779b97f4a7c15ULL;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

static void* work(void* arg) {
  Job* j = (Job*)arg;
  for (uint64_t i = j->lo; i < j->hi; ++i) {
    const uint32_t bits = index_to_bits(i);
    float x;
    memcpy(&x, &bits, 4);
    const long double e = expl((long double)x);
    const float ref = (float)e;
    {
      const float a = (float)(e * (1.0L - 0x1p-60L));
      const float b = (float)(e * (1.0L + 0x1p-60L));
      if (a != b) j->amb.push_back(bits);
    }
    const double y = nls::expf_as_double(x);
    const double yt = nls::expf_as_double_t(x, nls::kExpfPow2J64);
    const double rel = fabs((double)(((long double)y - e) / e));
    const double relt = fabs((double)(((long double)yt - e) / e));
    if (rel > j->max_rel) j->max_rel = rel;
    if (relt > j->max_rel_t) j->max_rel_t = relt;
    if (j->mode == 0) {
      if (nls::expf_is_hard(y) || nls::expf_is_hard(yt)) {
        j->hard_in.push_back(bits);
        uint32_t rb;
        memcpy(&rb, &ref, 4);
        j->hard_out.push_back(rb);
      } else if ((float)y != ref || (float)yt != ref) {
        j->mismatches++;
      }
    } else {
      const float got = nls::expf_cr(x);
      const float gott = nls::expf_cr_t(x, nls::kExpfPow2J64);
      uint32_t gb, gbt, rb;
      memcpy(&gb, &got, 4);
      memcpy(&gbt, &gott, 4);
      memcpy(&rb, &ref, 4);
      if (gb != rb || gbt != rb) j->mismatches++;
      j->checksum += mix(((uint64_t)bits << 32) | gb);
      j->checksum_t += mix(((uint64_t)bits << 32) | gbt);
    }
    j->count++;
  }
  return nullptr;
}

int main(int argc, char** argv) {
  const int mode = (argc > 1 && strcmp(argv[1], "verify") == 0) ? 1 : 0;
  const char* out_path = argc > 2 ? argv[2] : "nls_expf_table.h";
  const uint64_t total = (uint64_t)(kNegEnd - 0x80000000u) + kPosEnd;
  int nt = 8;
  if (getenv("NLS_SCAN_THREADS")) nt = atoi(getenv("NLS_SCAN_THREADS"));
  std::vector<Job> jobs(nt);
  std::vector<pthread_t> th(nt);
  for (int t = 0; t < nt; ++t) {
    jobs[t].lo = total * t / nt;
    jobs[t].hi = total * (t + 1) / nt;
    jobs[t].mode = mode;
    pthread_create(&th[t], nullptr, work, &jobs[t]);
  }
  std::vector<std::pair<uint32_t, uint32_t>> hard;
  std::vector<uint32_t> amb;
  uint64_t mism = 0, checksum = 0, checksum_t = 0, count = 0;
  double max_rel = 0, max_rel_t = 0;
  for (int t = 0; t < nt; ++t) {
    pthread_join(th[t], nullptr);
    for (size_t q = 0; q < jobs[t].hard_in.size(); ++q)
      hard.emplace_back(jobs[t].hard_in[q], jobs[t].hard_out[q]);
    amb.insert(amb.end(), jobs[t].amb.begin(), jobs[t].amb.end());
    mism += jobs[t].mismatches;
    checksum += jobs[t].checksum;
    checksum_t += jobs[t].checksum_t;
    count += jobs[t].count;
    max_rel = std::max(max_rel, jobs[t].max_rel);
    max_rel_t = std::max(max_rel_t, jobs[t].max_rel_t);
  }
  std::sort(hard.begin(), hard.end());
  printf("inputs %llu max_rel_err %.3e (2^%.2f) table form %.3e (2^%.2f) hard %zu mismatches %llu "
         "expl_ambiguous %zu\n",
         (unsigned long long)count, max_rel, log2(max_rel), max_rel_t, log2(max_rel_t), hard.size(),
         (unsigned long long)mism, amb.size());
  for (uint32_t b : amb) printf("expl_ambiguous 0x%08x\n", b);
  if (mode == 1) {
    printf("checksum 0x%016llx table form 0x%016llx\n", (unsigned long long)checksum,
           (unsigned long long)checksum_t);
    return mism != 0 || checksum != checksum_t;
  }
  FILE* f = fopen(out_path, "w");
  fprintf(f,
          "// Generated by nls_expf_scan.c++ (exhaustive scan of binary32 inputs in\n"
          "// (-104, 89)).  Inputs where either float64 evaluation in nls_expf.h lies too\n"
          "// close to a binary32 rounding boundary, with the correctly rounded\n"
          "// result of exp(x) (from a 64-bit-significand evaluation).  Sorted.\n"
          "#pragma once\n#include <stdint.h>\n#define NLS_EXPF_HARD_COUNT %zu\n"
          "namespace nls {\nconstexpr uint32_t kExpfHardInputs[%zu] = {\n",
          hard.size() ? hard.size() : 1, hard.size() ? hard.size() : 1);
  for (size_t q = 0; q < hard.size(); ++q)
    fprintf(f, "0x%08xu,%s", hard[q].first, (q % 6 == 5) ? "\n" : " ");
  if (hard.empty()) fprintf(f, "0xffffffffu");
  fprintf(f, "};\nconstexpr uint32_t kExpfHardResults[%zu] = {\n", hard.size() ? hard.size() : 1);
  for (size_t q = 0; q < hard.size(); ++q)
    fprintf(f, "0x%08xu,%s", hard[q].second, (q % 6 == 5) ? "\n" : " ");
  if (hard.empty()) fprintf(f, "0u");
  fprintf(f, "};\n}  // namespace nls\n");
  fclose(f);
  return mism != 0;
}
