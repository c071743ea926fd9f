// Host-only robustness check of the checkpoint reader and upload plan
// (krea2-hrx_amd/csrc/k2w8_checkpoint.cpp), built with AddressSanitizer and
// UndefinedBehaviorSanitizer by tests/test_checkpoint_fuzz.py. Two modes:
//   checkpoint_fuzz --mutate BASE ITERATIONS SEED: byte-level mutations of a valid
//     checkpoint (header bytes, JSON punctuation, the length prefix, truncation,
//     deletions and insertions), each written to a temporary file and run through
//     open -> tensor lookups -> plan -> span queries;
//   checkpoint_fuzz --files F...: the same calls on each given file.
// A sanitizer report aborts the process; otherwise it prints how many variants
// opened and planned.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "krea2_w8a8.h"

// The library's error channel and shape rule, which the reader calls (k2w8_api.cpp).
int k2w8_fail_invalid(const char *) { return K2W8_INVALID_ARGUMENT; }
int k2w8_fail_runtime(const char *, hipError_t) { return K2W8_RUNTIME; }
int k2w8_succeed() { return K2W8_OK; }
extern "C" int64_t k2w8_shape_gemm_pitch(int64_t k) { return k % 8192 == 0 ? k + 64 : k; }

namespace {

int g_opened = 0, g_planned = 0;

void exercise(const char *path) {
  k2w8_checkpoint *ck = nullptr;
  if (k2w8_checkpoint_open(path, &ck) != K2W8_OK) return;
  ++g_opened;
  (void)k2w8_checkpoint_block_count(ck);
  for (const char *name : {"blocks.0.attn.wq.weight", "blocks.0.mlp.up.weight_scale", "missing", ""}) {
    k2w8_tensor t;
    (void)k2w8_checkpoint_tensor(ck, name, &t);
  }
  k2w8_plan *plan = nullptr;
  if (k2w8_plan_for_checkpoint(ck, &plan) == K2W8_OK) {
    ++g_planned;
    (void)k2w8_plan_total_bytes(plan);
    (void)k2w8_plan_layers(plan);
    (void)k2w8_plan_span_count(plan);
    for (const char *name : {"blocks.0.qkvg", "blocks.0.gu", "blocks.0.down", "missing"}) {
      k2w8_span s;
      (void)k2w8_plan_span(plan, name, &s);
    }
    k2w8_plan_free(plan);
  }
  k2w8_checkpoint_close(ck);
}

std::vector<unsigned char> slurp(const char *path) {
  FILE *f = fopen(path, "rb");
  if (!f) abort();
  std::vector<unsigned char> v;
  fseek(f, 0, SEEK_END);
  v.resize((size_t)ftell(f));
  fseek(f, 0, SEEK_SET);
  if (fread(v.data(), 1, v.size(), f) != v.size()) abort();
  fclose(f);
  return v;
}

}  // namespace

int main(int argc, char **argv) {
  if (argc >= 2 && std::string(argv[1]) == "--files") {
    for (int i = 2; i < argc; ++i) exercise(argv[i]);
    printf("files %d opened %d planned %d\n", argc - 2, g_opened, g_planned);
    return 0;
  }
  if (argc != 6 || std::string(argv[1]) != "--mutate") {
    fprintf(stderr, "usage: %s --mutate BASE ITERATIONS SEED TMPFILE | --files F...\n", argv[0]);
    return 2;
  }
  const std::vector<unsigned char> base = slurp(argv[2]);
  const int iterations = atoi(argv[3]);
  std::mt19937_64 rng(strtoull(argv[4], nullptr, 10));
  const char *tmp = argv[5];
  uint64_t header = 0;
  memcpy(&header, base.data(), 8);
  static const char kPunct[] = "0123456789[]{},:\"-.eE ";
  for (int it = 0; it < iterations; ++it) {
    std::vector<unsigned char> v = base;
    const int kind = (int)(rng() % 8), edits = 1 + (int)(rng() % 8);
    for (int j = 0; j < edits && v.size() >= 16; ++j) {
      const size_t present = std::min<size_t>(header, v.size() - 8);
      const size_t at = 8 + rng() % present;
      switch (kind) {
        case 0: v[at] = (unsigned char)rng(); break;
        case 1: v[at] = (unsigned char)kPunct[rng() % (sizeof kPunct - 1)]; break;
        case 2: v[rng() % 8] = (unsigned char)rng(); break;
        case 3: v.resize(rng() % v.size()); break;
        case 4: {
          const uint64_t len = rng() % (header * 2 + 16);
          memcpy(v.data(), &len, 8);
          break;
        }
        case 5:
          for (size_t d = 0; d < 6 && at + d < v.size(); ++d) v[at + d] = '9';
          break;
        case 6: v.erase(v.begin() + at, v.begin() + std::min(v.size(), at + 1 + rng() % 16)); break;
        default: v.insert(v.begin() + at, (unsigned char)"\"a\":1,"[rng() % 6]); break;
      }
    }
    FILE *f = fopen(tmp, "wb");
    if (!f) abort();
    fwrite(v.data(), 1, v.size(), f);
    fclose(f);
    exercise(tmp);
  }
  printf("mutations %d opened %d planned %d\n", iterations, g_opened, g_planned);
  return 0;
}
