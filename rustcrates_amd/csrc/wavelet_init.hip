// wavelet_init.hip — EmbeddingLayer::create_embedding (embedding_layer.rs:
// 65-77) on gfx950: every token's embedding is a draw of src_dim values
// uniform in [-0.4, 0.5), decomposed by decompose_in_wavelet_2d_default
// (network_types/wavelet_network.rs:42-135), whose first CWT scale's row is
// the embedding.  The reference draws from the unseeded rand::rng(); here the
// draw is the project's counter generator on stream (layer << 12) | 0xFFF,
// index token * src_dim + k.
//
// The decomposition of a one-row input, with DB1 and SYMMETRIC padding:
//   each level: dwt_2d_full (wavelet_transform/dwt.rs:20-34) -- dwt_1d of the
//   row, whose low half at an even width w is (0 + x[2i] lo0) + x[2i+1] lo1,
//   then dwt_1d of every one-element column, whose low value is
//   (0 + l lo0) + l lo1 -- keeping the LL quadrant (get_ll_hl_lh_hh,
//   dwt.rs:379-401), for at most 5 levels and stopping before a level whose
//   transformed width is under 28 (wavelet_network.rs:97-102);
//   then the CMOR CWT at scale 2 (cwt_complex.rs:195-211): the full
//   convolution with the wavelet's scaled integral (utils/array_complex.rs:
//   38-149), -sqrt(2) times its successive differences, the centre w of them.
// The integral depends only on the wavelet and the scale, so the host forms
// it once per call (glibc cos, sin, pow, as Rust's f64 methods on Linux);
// one block per token does the rest.  Built with -ffp-contract=off: every
// multiply and add rounds on its own, in the reference's order.
#include <cmath>
#include <vector>

#include "kernels.hpp"

namespace mitok {

constexpr int EW_LEVELS = 5, EW_MIN_WIDTH = 28;  // DECOMPOSITION_LEVELS, min_width (wavelet_network.rs:13,48)
constexpr double EW_SCALE = 2.0, EW_FB = 1.5, EW_FC = 1.0;  // the first of scales 2, 8, 16, 32; CMOR fb, fc

// The CMOR wavelet's cumulative integral at the scale, reversed
// (integrate_complex): x = linspace_complex(-8, 8, 1024, true) (the step
// added point by point, the end set exactly), y = cmorl(x) =
// cos(2 pi fc x) E^(-x^2 / fb) / sqrt(pi fb) - i sin(...) E^(...) / sqrt(pi fb)
// (cwt_type_resolver.rs:114-123; E.powf is pow with base e), the running sum
// of y * step, sampled at index floor(v / (scale * step)) for v = 0, 1, ...,
// scale * 16 (arange, utils/array.rs:8-20).
static int cmor_scaled_integral(double scale, double fb, double fc, std::vector<double2>& k) {
  constexpr int NP = 1024;  // 2^10 points (wavefun_complex, cwt_complex.rs:268-289)
  std::vector<double> xs(NP);
  const double start = -8.0, end = 8.0, span = end - start;
  const double step_ls = span / ((double)NP - 1.0);
  double t = start;
  for (int i = 0; i < NP; ++i) {
    xs[i] = t;
    t = t + step_ls;
  }
  xs[NP - 1] = end;
  const double step = xs[1] - xs[0];
  std::vector<double2> integral(NP);
  for (int i = 0; i < NP; ++i) {
    const double re = xs[i];
    const double ang = 2.0 * M_PI * fc * re;
    const double g = std::pow(M_E, -std::pow(re, 2.0) / fb);
    const double den = std::sqrt(M_PI * fb);
    const double yr = std::cos(ang) * g / den, yi = -1.0 * (std::sin(ang) * g / den);
    double2 sum = make_double2(yr * step, yi * step);
    if (i > 0) sum = make_double2(sum.x + integral[i - 1].x, sum.y + integral[i - 1].y);
    integral[i] = sum;
  }
  const double range = xs[NP - 1] - xs[0];
  const double a_end = scale * range + 1.0;
  const size_t K = (size_t)((a_end - 0.0) / 1.0);
  k.assign(K, make_double2(0.0, 0.0));
  double v = 0.0;
  for (size_t j = 0; j < K; ++j) {
    const size_t idx = (size_t)(v / (scale * step));
    if (idx >= (size_t)NP) return ERR_ARG;
    k[K - 1 - j] = integral[idx];
    v = v + 1.0;
  }
  return OK;
}

// width after the decomposition of a src-wide row (0: src is not supported)
int embedding_wavelet_dim(int src) {
  if (src < 2 || src > EW_MAX_SRC || (src & (src - 1)) != 0) return 0;  // even widths at every level
  int w = src;
  for (int lv = 0; lv < EW_LEVELS; ++lv) {
    if (w < EW_MIN_WIDTH) break;  // the transformed width of a one-row input is w
    w >>= 1;
  }
  return w;
}

__device__ __forceinline__ double2 cmul_ref(double2 a, double2 b) {
  return make_double2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}

// one block of 64 threads per token; LDS: two rows of src doubles
__global__ __launch_bounds__(64) void k_embedding_wavelet(double2* __restrict__ table, int dim, int src,
                                                          const double2* __restrict__ kern, int K, uint64_t key,
                                                          double lo0, double lo1) {
  extern __shared__ double ew_buf[];
  double* a = ew_buf;
  double* b = ew_buf + src;
  const int lane = threadIdx.x;
  const long tok = blockIdx.x;
  const double lo = -0.4, hi = 0.5;
  for (int k = lane; k < src; k += 64) {
    const double u = (double)(mix64(key ^ (uint64_t)(tok * src + k)) >> 11) * 0x1.0p-53;
    a[k] = lo + (hi - lo) * u;
  }
  __syncthreads();
  int w = src;
  for (int lv = 0; lv < EW_LEVELS; ++lv) {
    if (w < EW_MIN_WIDTH) break;
    for (int i = lane; i < w / 2; i += 64) {
      const double l = (0.0 + a[2 * i] * lo0) + a[2 * i + 1] * lo1;
      b[i] = (0.0 + l * lo0) + l * lo1;
    }
    __syncthreads();
    double* t = a;
    a = b;
    b = t;
    w >>= 1;
  }
  // convolve_complex(row, kernel, FULL): the shorter operand reversed over the
  // longer one padded by (nout - longer) zeros on each side, summed in order
  const int n = w, nout = n + K - 1;
  const bool kshort = K < n;
  const int ls = kshort ? K : n, ll = kshort ? n : K;
  const int pad = nout - ll, flen = ll + 2 * pad;
  const double ss = -1.0 * sqrt(EW_SCALE);
  const int down = (int)floor((double)(nout - 1 - n) / 2.0);
  for (int t = lane; t < n; t += 64) {
    double2 c2[2];
    for (int q = 0; q < 2; ++q) {
      const int j = down + t + q;
      double2 sum = make_double2(0.0, 0.0);
      for (int i = 0; i < ls; ++i) {
        const int m = (i + j) % flen;
        const int li = m - pad;
        double2 f;  // the padded longer operand
        if (li < 0 || li >= ll) f = make_double2(0.0, 0.0);
        else f = kshort ? make_double2(a[li], 0.0) : kern[li];
        const int si = ls - 1 - i;  // the shorter operand, reversed
        const double2 s = kshort ? kern[si] : make_double2(a[si], 0.0);
        const double2 p = cmul_ref(f, s);
        sum = make_double2(sum.x + p.x, sum.y + p.y);
      }
      c2[q] = sum;
    }
    // get_coef_complex: -sqrt(scale) (conv[j + 1] - conv[j])
    const double2 d = make_double2(c2[1].x - c2[0].x, c2[1].y - c2[0].y);
    table[tok * dim + t] = make_double2(ss * d.x, ss * d.y);
  }
}

int embedding_wavelet_init(hipStream_t st, double2* table, int vocab, int dim, int src, uint64_t key,
                           double2* kern_d, size_t kern_cap) {
  if (embedding_wavelet_dim(src) != dim || vocab <= 0) return ERR_ARG;
  std::vector<double2> kern;
  if (cmor_scaled_integral(EW_SCALE, EW_FB, EW_FC, kern) != OK) return ERR_ARG;
  if (kern.size() > kern_cap) return ERR_ARG;
  if (hipMemcpyAsync(kern_d, kern.data(), kern.size() * sizeof(double2), hipMemcpyHostToDevice, st) != hipSuccess)
    return ERR_HIP;
  // DB1's low-pass filter: 1/sqrt(2) twice (dwt_coeffients.rs DB_1)
  const double c = 0x1.6a09e667f3bcdp-1;  // 0.7071067811865476, 1/sqrt(2) correctly rounded
  MITOK_LAUNCH(k_embedding_wavelet, dim3((unsigned)vocab), dim3(64), (unsigned)(2 * src * sizeof(double)), st, table,
               dim, src, (const double2*)kern_d, (int)kern.size(), key, c, c);
  // the host vector must outlive the copy
  if (hipStreamSynchronize(st) != hipSuccess) return ERR_HIP;
  return OK;
}

}  // namespace mitok
