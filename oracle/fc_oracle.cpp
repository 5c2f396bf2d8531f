// CPU oracle of the flashcodec KV-codec hot path — TEST INFRASTRUCTURE ONLY.
//
// Scalar restatement of the reference algorithm (flashcodec-kv 1.0.0) used by
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
// checker of the HIP kernels; nothing in the flashcodec_amd package links,
// loads or calls it.  It shares no source with the package.
//
// Values travel as fp32 arrays holding values exactly representable in the
// stream dtype (fp32, fp16 or bf16); `dtype` (0 fp32, 1 fp16, 2 bf16) says
// which rounding applies where the reference casts.  Each function names
// the reference lines it restates.  The arithmetic order is the one the
// reference's CPU PyTorch path executes (pinned by the golden vectors under
// tests/golden/):
//   * dct_compress (flashcodec/codecs/jpeg.py:55-67): the fp32 GEMM
//     accumulates each output as a fused multiply-add chain over the taps in
//     order, starting from zero; the result is cast to the input dtype.
//   * dct_decompress (jpeg.py:70-82): same chain over the coefficients.
//   * quantize_coeffs (jpeg.py:85-100): absmax in the coefficient dtype,
//     scale = dtype(absmax / 127.0f), 1 where not > 0, codes =
//     round-half-even(c / scale) clamped to +-127.
//   * png_filter (flashcodec/codecs/png.py:36-60): fp32 deltas; Top-M by
//     |delta| through std::nth_element over (value, index) pairs with a
//     "NaN first, then larger" comparator (what torch.topk runs on the CPU);
//     pruned deltas multiplied by 0.
//   * png_reconstruct (png.py:63-74): torch's CPU cumsum of float
//     accumulates in double and rounds each prefix to float.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <utility>
#include <vector>

namespace {

uint32_t bits_of(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}
float float_of(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// fp32 -> fp16 -> fp32, round to nearest even, subnormals and overflow
// handled as IEEE binary16.
float round_f16(float f) {
  if (std::isnan(f)) return f;
  const double a = std::fabs((double)f);
  if (a == 0.0) return f;
  if (a >= 65520.0) return std::copysign(INFINITY, f);  // rounds past max half
  int e;
  std::frexp(a, &e);  // a = m * 2^e, m in [0.5, 1)
  // spacing of binary16 at this magnitude: 2^(e-11), at least 2^-24
  int q = e - 11;
  if (q < -24) q = -24;
  const double step = std::ldexp(1.0, q);
  double n = a / step;  // exact: a has 24 significant bits, step is a power of 2
  double fl = std::floor(n);
  double rem = n - fl;
  if (rem > 0.5 || (rem == 0.5 && std::fmod(fl, 2.0) != 0.0)) fl += 1.0;
  return (float)std::copysign(fl * step, (double)f);
}

// fp32 -> bf16 -> fp32, round to nearest even (NaN kept as NaN).
float round_bf16(float f) {
  if (std::isnan(f)) return f;
  uint32_t u = bits_of(f);
  const uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return float_of(u & 0xffff0000u);
}

float round_to(int dtype, float f) {
  switch (dtype) {
    case 1: return round_f16(f);
    case 2: return round_bf16(f);
    default: return f;
  }
}

// int8 code of a rounded quotient q: clamp to [-127, 127]
// (quantize_coeffs, flashcodec/codecs/jpeg.py:96-99).  The reference casts
// a NaN quotient to int8, which C++ leaves undefined; x86's truncating
// conversion gives 0 there, and 0 is the code used here.
int8_t quant_clamp(float q) {
  if (std::isnan(q)) return 0;
  return (int8_t)std::min(127.0f, std::max(-127.0f, q));
}

}  // namespace

extern "C" {

float orc_round(int dtype, float f) { return round_to(dtype, f); }

// dct_compress + quantize_coeffs on items of r rows x D features.
// x: (n_items, r, D) input values; basis: k x r fp32.
// coef: (n_items, k, D) coefficients (values of the input dtype).
// When quant: codes (n_items, k, D), scales (n_items, k).
void orc_jpeg_encode(const float* x, long n_items, int r, int k, long D, const float* basis,
                     int dtype, int quant, float* coef, int8_t* codes, float* scales) {
  for (long it = 0; it < n_items; ++it) {
    const float* xb = x + it * r * D;
    float* cb = coef + it * k * D;
    for (int j = 0; j < k; ++j) {
      for (long d = 0; d < D; ++d) {
        float acc = 0.0f;
        for (int t = 0; t < r; ++t) acc = std::fmaf(xb[t * D + d], basis[j * r + t], acc);
        cb[j * D + d] = round_to(dtype, acc);
      }
      if (!quant) continue;
      float amax = 0.0f;
      for (long d = 0; d < D; ++d) amax = std::max(amax, std::fabs(cb[j * D + d]));
      float s = round_to(dtype, amax / 127.0f);
      if (!(s > 0.0f)) s = 1.0f;
      scales[it * k + j] = s;
      for (long d = 0; d < D; ++d) {
        const float q = std::nearbyint(cb[j * D + d] / s);  // default mode: ties to even
        codes[(it * k + j) * D + d] = quant_clamp(q);
      }
    }
  }
}

// dequantize_coeffs(q, scale, dtype) on rows of D codes.
void orc_dequantize(const int8_t* codes, const float* scales, long n_rows, long D, int dtype,
                    float* out) {
  for (long i = 0; i < n_rows; ++i) {
    const float s = round_to(dtype, scales[i]);
    for (long d = 0; d < D; ++d) out[i * D + d] = round_to(dtype, (float)codes[i * D + d] * s);
  }
}

// quantize_coeffs on rows of D coefficient values of `dtype`.
void orc_quantize(const float* c, long n_rows, long D, int dtype, int8_t* codes, float* scales) {
  for (long i = 0; i < n_rows; ++i) {
    float amax = 0.0f;
    for (long d = 0; d < D; ++d) amax = std::max(amax, std::fabs(c[i * D + d]));
    float s = round_to(dtype, amax / 127.0f);
    if (!(s > 0.0f)) s = 1.0f;
    scales[i] = s;
    for (long d = 0; d < D; ++d) {
      const float q = std::nearbyint(c[i * D + d] / s);
      codes[i * D + d] = quant_clamp(q);
    }
  }
}

// dct_decompress of items (k coefficient rows of D) into r rows.
// quant: coefficients are codes * scales (fp32), else `coef` values.
// out: (n_items, r, D), rounded to out_dtype.
void orc_jpeg_decode(const float* coef, const int8_t* codes, const float* scales, int quant,
                     long n_items, int r, int k, long D, const float* basis, int out_dtype,
                     float* out) {
  std::vector<float> deq((size_t)k * D);
  for (long it = 0; it < n_items; ++it) {
    for (int j = 0; j < k; ++j)
      for (long d = 0; d < D; ++d)
        deq[j * D + d] = quant ? (float)codes[(it * k + j) * D + d] * scales[it * k + j]
                               : coef[(it * k + j) * D + d];
    for (int t = 0; t < r; ++t)
      for (long d = 0; d < D; ++d) {
        float acc = 0.0f;
        for (int j = 0; j < k; ++j) acc = std::fmaf(deq[j * D + d], basis[j * r + t], acc);
        out[(it * r + t) * D + d] = round_to(out_dtype, acc);
      }
  }
}

// Selection of torch's CPU topk(m) (largest) over n values: returns a keep
// mask.  torch partial-sorts when m * 64 <= n, else nth_element.
void orc_topk_keep(const float* v, int n, int m, uint8_t* keep) {
  std::vector<std::pair<double, int64_t>> q((size_t)n);
  for (int i = 0; i < n; ++i) q[i] = {(double)v[i], (int64_t)i};
  auto comp = [](const std::pair<double, int64_t>& a, const std::pair<double, int64_t>& b) {
    return (std::isnan(a.first) && !std::isnan(b.first)) || (a.first > b.first);
  };
  if ((int64_t)m * 64 <= n)
    std::partial_sort(q.begin(), q.begin() + m, q.end(), comp);
  else
    std::nth_element(q.begin(), q.begin() + (m - 1), q.end(), comp);
  for (int i = 0; i < n; ++i) keep[i] = 0;
  for (int i = 0; i < m; ++i) keep[q[i].second] = 1;
}

// png_filter on items of r rows: anchors (n_items, D), deltas
// (n_items, r-1, D).  keep_m == 0: no pruning.
void orc_png_encode(const float* x, long n_items, int r, long D, int keep_m, float* deltas,
                    float* anchors) {
  const int n = r - 1;
  std::vector<float> col((size_t)n);
  std::vector<uint8_t> keep((size_t)n);
  for (long it = 0; it < n_items; ++it) {
    const float* xb = x + it * r * D;
    float* db = deltas + it * n * D;
    for (long d = 0; d < D; ++d) {
      anchors[it * D + d] = xb[d];
      for (int i = 0; i < n; ++i) db[i * D + d] = xb[(i + 1) * D + d] - xb[i * D + d];
      if (keep_m > 0 && keep_m < n + 1) {
        for (int i = 0; i < n; ++i) col[i] = std::fabs(db[i * D + d]);
        orc_topk_keep(col.data(), n, std::min(keep_m, n), keep.data());
        for (int i = 0; i < n; ++i)
          if (!keep[i]) db[i * D + d] = db[i * D + d] * 0.0f;
      }
    }
  }
}

// png_reconstruct: out (n_items, r, D) in `dtype`.
void orc_png_decode(const float* deltas, const float* anchors, long n_items, int r, long D,
                    int dtype, float* out) {
  const int n = r - 1;
  for (long it = 0; it < n_items; ++it)
    for (long d = 0; d < D; ++d) {
      const float base = anchors[it * D + d];
      out[(it * r) * D + d] = round_to(dtype, base);
      double run = 0.0;
      for (int i = 0; i < n; ++i) {
        run += (double)deltas[(it * n + i) * D + d];
        out[(it * r + i + 1) * D + d] = round_to(dtype, base + (float)run);
      }
    }
}

// Decode attention in double precision, by definition: every archived block
// is synthesised as tokens = A @ rows (A: r x s), then one softmax over all
// archived and raw tokens (flashcodec/attention.py:64-140).
//   q: (B, Hq, D); rows_k/rows_v: (B, Hkv, nb, s, D) dequantised rows;
//   raw_k/raw_v: (B, Hkv, nr, D); out: (B, Hq, D).
void orc_attention(const double* q, const double* rows_k, const double* rows_v,
                   const double* raw_k, const double* raw_v, const double* A, long B, long Hq,
                   long Hkv, long nb, int r, int s, long nr, long D, double scale, double* out,
                   int n_threads) {
  const long G = Hq / Hkv;
  const long S = nb * r + nr;
#pragma omp parallel for schedule(dynamic) num_threads(n_threads)
  for (long bq = 0; bq < B * Hq; ++bq) {
    const long b = bq / Hq, hq = bq % Hq, hk = hq / G;
    const double* qv = q + bq * D;
    std::vector<double> logit((size_t)(S > 0 ? S : 1));
    std::vector<double> tok((size_t)D);
    const long base = (b * Hkv + hk);
    double mx = -INFINITY;
    for (long n = 0; n < nb; ++n) {
      const double* rk = rows_k + (base * nb + n) * s * D;
      for (int p = 0; p < r; ++p) {
        double acc = 0.0;
        for (long d = 0; d < D; ++d) {
          double kv = 0.0;
          for (int j = 0; j < s; ++j) kv += A[p * s + j] * rk[j * D + d];
          acc += qv[d] * kv;
        }
        logit[n * r + p] = acc * scale;
        mx = std::max(mx, logit[n * r + p]);
      }
    }
    for (long t = 0; t < nr; ++t) {
      const double* kr = raw_k + (base * nr + t) * D;
      double acc = 0.0;
      for (long d = 0; d < D; ++d) acc += qv[d] * kr[d];
      logit[nb * r + t] = acc * scale;
      mx = std::max(mx, logit[nb * r + t]);
    }
    double l = 0.0;
    for (long i = 0; i < S; ++i) {
      logit[i] = std::exp(logit[i] - mx);
      l += logit[i];
    }
    double* o = out + bq * D;
    for (long d = 0; d < D; ++d) o[d] = 0.0;
    for (long n = 0; n < nb; ++n) {
      const double* rv = rows_v + (base * nb + n) * s * D;
      for (int p = 0; p < r; ++p) {
        const double w = logit[n * r + p] / l;
        for (long d = 0; d < D; ++d) {
          double vv = 0.0;
          for (int j = 0; j < s; ++j) vv += A[p * s + j] * rv[j * D + d];
          o[d] += w * vv;
        }
      }
    }
    for (long t = 0; t < nr; ++t) {
      const double* vr = raw_v + (base * nr + t) * D;
      const double w = logit[nb * r + t] / l;
      for (long d = 0; d < D; ++d) o[d] += w * vr[d];
    }
  }
}

}  // extern "C"
