// Host build of the kernels' exp (marian-edge_amd/csrc/ref_expf.h) compared
// with the C library's expf, which the reference's f32::exp calls, on every
// fp32 input with bit pattern = start (mod stride).  Prints the count of
// inputs checked and of mismatching results; exits 1 on any mismatch.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "ref_expf.h"

int main(int argc, char** argv) {
  const long long stride = argc > 1 ? atoll(argv[1]) : 1;
  static const uint64_t tab[32] = {MH_EXP2_TABLE_32};
  long long checked = 0, bad = 0, first_bad = -1;
#pragma omp parallel for reduction(+ : checked, bad) schedule(static, 1 << 16)
  for (long long u = 0; u < (1LL << 32); u += stride) {
    float x;
    const uint32_t ux = (uint32_t)u;
    std::memcpy(&x, &ux, 4);
    const float want = expf(x), got = mh::ref_expf(x, tab);
    uint32_t wb, gb;
    std::memcpy(&wb, &want, 4);
    std::memcpy(&gb, &got, 4);
    ++checked;
    if (wb != gb && !(want != want && got != got)) {
      ++bad;
#pragma omp critical
      if (first_bad < 0) first_bad = u;
    }
  }
  std::printf("checked %lld mismatches %lld first 0x%llx\n", checked, bad,
              (unsigned long long)(first_bad < 0 ? 0 : first_bad));
  return bad ? 1 : 0;
}
