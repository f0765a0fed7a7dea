// The decode step's deferred argmax word (lm_pack_key / lm_key_row in
// csrc/model_kernels.hpp): workgroups each pick their best (value, row) with
// the kernels' comparison (higher value, then lower row; NaN and -inf never
// win from the starting -FLT_MAX), pack it, and an atomic max folds the
// words.  The folded word's row must be the row a sequential pass of that
// comparison picks over the whole vocabulary, 0 when no row wins, for any
// split into workgroups.  Brute force over random vectors with NaN, +-inf,
// +-0, +-FLT_MAX, denormals and planted ties.
#include <cfloat>
#include <climits>
#include <cmath>
#include <cstdio>
#include <random>
#include <vector>

#include "model_kernels.hpp"

namespace {
bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }
}  // namespace

int main() {
  std::mt19937 rng(20261202);
  const float specials[] = {NAN, INFINITY, -INFINITY, 0.0f, -0.0f, FLT_MAX, -FLT_MAX,
                            1.0f, -1.0f, 1e-40f, -1e-40f, 3.5f};
  const int nspecial = sizeof(specials) / sizeof(specials[0]);
  int fails = 0;
  for (int trial = 0; trial < 200000; ++trial) {
    const int n = 1 + static_cast<int>(rng() % 12);
    std::vector<float> v(n);
    for (int i = 0; i < n; ++i) {
      switch (rng() % 4) {
        case 0: v[i] = specials[rng() % nspecial]; break;
        case 1: v[i] = static_cast<float>(static_cast<int>(rng() % 5) - 2); break;  // ties
        default:
          v[i] = std::ldexp(static_cast<float>(rng() % 1000) - 500.0f,
                            static_cast<int>(rng() % 40) - 20);
      }
    }
    float bv = -FLT_MAX;
    int bi = INT_MAX;
    for (int i = 0; i < n; ++i) {
      if (better(v[i], i, bv, bi)) {
        bv = v[i];
        bi = i;
      }
    }
    const int expect = bi == INT_MAX ? 0 : bi;
    unsigned long long folded = 0;
    for (int start = 0; start < n;) {
      int len = 1 + static_cast<int>(rng() % 4);
      if (start + len > n) len = n - start;
      float cv = -FLT_MAX;
      int ci = INT_MAX;
      for (int i = start; i < start + len; ++i) {
        if (better(v[i], i, cv, ci)) {
          cv = v[i];
          ci = i;
        }
      }
      // as lm_head_decode_kernel: a workgroup with no winning row offers its
      // first row at the lowest key
      const unsigned long long k =
          ci == INT_MAX ? qlin::lm_pack_key(NAN, start) : qlin::lm_pack_key(cv, ci);
      if (k > folded) folded = k;
      start += len;
    }
    if (!(folded >> 63) || qlin::lm_key_row(folded) != expect) {
      if (fails < 5) std::printf("trial %d: expected row %d, got %d\n", trial, expect,
                                 qlin::lm_key_row(folded));
      ++fails;
    }
  }
  // the largest row a 31-bit field holds, and row 0
  if (qlin::lm_key_row(qlin::lm_pack_key(1.0f, 0x7FFFFFFE)) != 0x7FFFFFFE ||
      qlin::lm_key_row(qlin::lm_pack_key(-1.0f, 0)) != 0) {
    ++fails;
  }
  std::printf("argmax key: %d failures\n", fails);
  return fails == 0 ? 0 : 1;
}
