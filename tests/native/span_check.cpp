// Host build of the span search in torchsplinekan_amd/csrc/kan_spline.h, for
// tests/test_span_search.py.  Reads "nk count" then, per case, nk knots and
// one x (all as doubles) from stdin, and prints per case the spans found by
// knot_span<float>, knot_span<double>, and lane 0 / lane 3 of a four-way
// knot_spans<4, float> call whose other lanes search other rows.
#include <cstdio>
#include <vector>

#include "kan_spline.h"

int main() {
  int nk = 0, count = 0;
  if (std::scanf("%d %d", &nk, &count) != 2) return 2;
  std::vector<double> td(nk);
  std::vector<float> tf(nk), other(nk);
  for (int c = 0; c < count; ++c) {
    for (int j = 0; j < nk; ++j) {
      if (std::scanf("%lf", &td[j]) != 1) return 2;
      tf[j] = (float)td[j];
      other[j] = (float)(nk - j);  // a descending row in the neighbouring lanes
    }
    double x = 0.0;
    if (std::scanf("%lf", &x) != 1) return 2;
    const float xf = (float)x;
    const float* rows[4] = {tf.data(), other.data(), other.data(), tf.data()};
    const float xs[4] = {xf, 0.5f, 1e9f, xf};
    int m4[4];
    kan::knot_spans<4, float>(rows, nk, xs, m4);
    std::printf("%d %d %d %d\n", kan::knot_span(tf.data(), nk, xf),
                kan::knot_span(td.data(), nk, x), m4[0], m4[3]);
  }
  return 0;
}
