// Host-side tests of the nspeech::rocm mirror (nspeech_amd/host/rocm_kernels.h),
// written the way the reference's Kokoro GPU self-tests are
// (src/kokoro/gpu_decoder.rs:64-456): deterministic known-answer inputs, the
// expected values from inline float64 formulas, a max-error report per test,
// plus a tolerance the reference's self-tests do not assert. Returns 0 when
// every test passes. Run on a GPU by tests/test_gpu_host_mirror.py.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "rocm_kernels.h"

using namespace nspeech::rocm;

namespace {

int g_failed = 0;

void report(const char* name, double err, double tol) {
  const bool ok = err <= tol;
  std::printf("%-34s max scaled error %.3e (tol %.0e) %s\n", name, err, tol, ok ? "ok" : "FAIL");
  if (!ok) ++g_failed;
}

void expect_throw(const char* name, const std::function<void()>& f, const char* needle) {
  try {
    f();
  } catch (const Error& e) {
    const bool ok = std::strstr(e.what(), needle) != nullptr;
    std::printf("%-34s threw \"%s\" %s\n", name, e.what(), ok ? "ok" : "FAIL");
    if (!ok) ++g_failed;
    return;
  }
  std::printf("%-34s did not throw FAIL\n", name);
  ++g_failed;
}

// IEEE half <-> float (round to nearest even), host side.
uint16_t f2h(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  int32_t e = (int32_t)((x >> 23) & 0xff) - 127 + 15;
  uint32_t m = x & 0x7fffffu;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    m |= 0x800000u;
    const int shift = 14 - e;
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;
  return (uint16_t)(sign | h);
}

float h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
  uint32_t x;
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-08f;
    std::memcpy(&x, &v, 4);
    x |= sign;
  } else if (e == 31) {
    x = sign | 0x7f800000u | (m << 13);
  } else {
    x = sign | ((e + 112) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

double scaled(double got, double ref) { return std::fabs(got - ref) / std::max(std::fabs(ref), 1.0); }

// Kokoro self-test inputs (gpu_decoder.rs:84-87): x[i] = sin(0.001 i) * 3,
// gamma_c = f16(sin(0.01c) * 0.5), beta_c = f16(cos(0.02c) * 0.3),
// alpha_c = f16(1 + sin(0.005c)).
void test_adain_snake_f32(const RocmDevice& dev, const RocmKernels& k, size_t C, size_t T, const char* name) {
  std::vector<float> x(C * T);
  for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin(0.001f * (float)i) * 3.0f;
  std::vector<uint16_t> g(C), b(C), a(C);
  for (size_t c = 0; c < C; ++c) {
    g[c] = f2h(std::sin(0.01f * (float)c) * 0.5f);
    b[c] = f2h(std::cos(0.02f * (float)c) * 0.3f);
    a[c] = f2h(1.0f + std::sin(0.005f * (float)c));
  }
  Tensor X = Tensor::from_host(dev, x.data(), {C, T}, DType::F32);
  Tensor G = Tensor::from_host(dev, g.data(), {C}, DType::F16);
  Tensor B = Tensor::from_host(dev, b.data(), {C}, DType::F16);
  Tensor A = Tensor::from_host(dev, a.data(), {C}, DType::F16);
  Tensor O = Tensor::empty(dev, {C, T}, DType::F32);
  RocmKokoroBackend be(dev, k);
  be.adain_snake_f32(X.buffer(), G.buffer(), B.buffer(), A.buffer(), O.buffer(), C, T);
  dev.synchronize();
  std::vector<float> o = O.to_vec<float>();
  double err = 0;
  for (size_t c = 0; c < C; ++c) {
    double mean = 0, var = 0;
    for (size_t t = 0; t < T; ++t) mean += x[c * T + t];
    mean /= (double)T;
    for (size_t t = 0; t < T; ++t) var += (x[c * T + t] - mean) * (x[c * T + t] - mean);
    var /= (double)T;
    const double al = h2f(a[c]);
    const double inv_a = (double)(1.0f / (h2f(a[c]) + 1e-9f));
    for (size_t t = 0; t < T; ++t) {
      const double y = (x[c * T + t] - mean) / std::sqrt(var + 1e-5) * (1.0 + h2f(g[c])) + h2f(b[c]);
      const double s = std::sin(al * y);
      err = std::max(err, scaled(o[c * T + t], y + s * s * inv_a));
    }
  }
  report(name, err, 1e-5);
}

void test_layernorm_std_f32in(const RocmDevice& dev, const RocmKernels& k) {
  const size_t R = 17, N = 640;  // decoder width of layernorm_standard_f32in_640
  std::vector<float> x(R * N);
  std::vector<uint16_t> w(N);
  for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin(0.1f * (float)i) * 3.0f + 0.5f;
  for (size_t c = 0; c < N; ++c) w[c] = f2h(1.0f + 0.1f * std::cos(0.03f * (float)c));
  Tensor X = Tensor::from_host(dev, x.data(), {R, N}, DType::F32);
  Tensor W = Tensor::from_host(dev, w.data(), {N}, DType::F16);
  Tensor O = Tensor::empty(dev, {R, N}, DType::F16);
  triton_layernorm_std_f32in(dev, k, X, W, O, R, N);
  dev.synchronize();
  std::vector<uint16_t> o = O.to_vec<uint16_t>();
  double err = 0;
  for (size_t r = 0; r < R; ++r) {
    double m = 0, v = 0;
    for (size_t c = 0; c < N; ++c) m += x[r * N + c];
    m /= N;
    for (size_t c = 0; c < N; ++c) v += (x[r * N + c] - m) * (x[r * N + c] - m);
    v /= N;
    for (size_t c = 0; c < N; ++c)
      err = std::max(err, scaled(h2f(o[r * N + c]), (x[r * N + c] - m) / std::sqrt(v + 1e-5) * h2f(w[c])));
  }
  report("triton_layernorm_std_f32in", err, 2e-3);
}

void test_layernorm_unit_offset_and_bare(const RocmDevice& dev, const RocmKernels& k) {
  const size_t R = 9, N = 768;  // encoder width of layernorm_unit_offset_768
  std::vector<uint16_t> x(R * N), g(N);
  for (size_t i = 0; i < x.size(); ++i) x[i] = f2h(std::sin(0.37f * (float)i) * 2.0f);
  for (size_t c = 0; c < N; ++c) g[c] = f2h(0.05f * std::sin(0.11f * (float)c));
  Tensor X = Tensor::from_host(dev, x.data(), {R, N}, DType::F16);
  Tensor G = Tensor::from_host(dev, g.data(), {N}, DType::F16);
  Tensor U = triton_layernorm_unit_offset(dev, k, X, G, R, N);
  Tensor Bo = triton_layernorm_bare(dev, k, X, R, N);
  dev.synchronize();
  std::vector<uint16_t> u = U.to_vec<uint16_t>(), bo = Bo.to_vec<uint16_t>();
  double eu = 0, eb = 0;
  for (size_t r = 0; r < R; ++r) {
    double m = 0, v = 0;
    for (size_t c = 0; c < N; ++c) m += h2f(x[r * N + c]);
    m /= N;
    for (size_t c = 0; c < N; ++c) v += (h2f(x[r * N + c]) - m) * (h2f(x[r * N + c]) - m);
    v /= N;
    for (size_t c = 0; c < N; ++c) {
      const double n = (h2f(x[r * N + c]) - m) / std::sqrt(v + 1e-5);
      eu = std::max(eu, scaled(h2f(u[r * N + c]), n * (h2f(g[c]) + 1.0)));
      eb = std::max(eb, scaled(h2f(bo[r * N + c]), n));
    }
  }
  report("triton_layernorm_unit_offset", eu, 2e-3);
  report("triton_layernorm_bare", eb, 2e-3);
}

void test_elementwise(const RocmDevice& dev, const RocmKernels& k) {
  const size_t n = 3000;
  std::vector<uint16_t> x(n), r(n), fc1(2 * n);
  for (size_t i = 0; i < n; ++i) {
    x[i] = f2h(std::sin(0.05f * (float)i) * 4.0f);
    r[i] = f2h(std::cos(0.07f * (float)i));
  }
  for (size_t i = 0; i < 2 * n; ++i) fc1[i] = f2h(std::sin(0.013f * (float)i) * 3.0f);
  Tensor X = Tensor::from_host(dev, x.data(), {n}, DType::F16);
  Tensor Rr = Tensor::from_host(dev, r.data(), {n}, DType::F16);
  Tensor F = Tensor::from_host(dev, fc1.data(), {2 * n}, DType::F16);
  Tensor Gl = triton_gelu(dev, k, X, n);
  Tensor Ad = triton_residual_add(dev, k, X, Rr, n);
  Tensor Gs = Tensor::empty(dev, {n}, DType::F16);
  triton_glu_silu(dev, k, F, Gs, n);
  dev.synchronize();
  std::vector<uint16_t> gl = Gl.to_vec<uint16_t>(), ad = Ad.to_vec<uint16_t>(), gs = Gs.to_vec<uint16_t>();
  double eg = 0, ea = 0, es = 0;
  for (size_t i = 0; i < n; ++i) {
    const double v = h2f(x[i]);
    eg = std::max(eg, scaled(h2f(gl[i]), v * 0.5 * (1.0 + std::erf(v / std::sqrt(2.0)))));
    ea = std::max(ea, scaled(h2f(ad[i]), (double)h2f(x[i]) + h2f(r[i])));
    const double gate = h2f(fc1[n + i]);
    es = std::max(es, scaled(h2f(gs[i]), gate / (1.0 + std::exp(-gate)) * h2f(fc1[i])));
  }
  report("triton_gelu", eg, 2e-3);
  report("triton_residual_add", ea, 2e-3);
  report("triton_glu_silu", es, 2e-3);
}

void test_residual_add_layernorm(const RocmDevice& dev, const RocmKernels& k) {
  const size_t R = 5, D = 640;
  std::vector<uint16_t> proj(R * D), w(D);
  std::vector<float> res(R * D);
  for (size_t i = 0; i < R * D; ++i) {
    proj[i] = f2h(std::sin(0.21f * (float)i));
    res[i] = std::cos(0.017f * (float)i) * 2.0f;
  }
  for (size_t c = 0; c < D; ++c) w[c] = f2h(1.0f + 0.2f * std::sin(0.05f * (float)c));
  Tensor P = Tensor::from_host(dev, proj.data(), {R, D}, DType::F16);
  Tensor Rs = Tensor::from_host(dev, res.data(), {R, D}, DType::F32);
  Tensor W = Tensor::from_host(dev, w.data(), {D}, DType::F16);
  Tensor H = Tensor::empty(dev, {R, D}, DType::F32);
  Tensor N = Tensor::empty(dev, {R, D}, DType::F16);
  triton_residual_add_layernorm(dev, k, P, Rs, H, W, N, R, D);
  dev.synchronize();
  std::vector<float> h = H.to_vec<float>();
  std::vector<uint16_t> nn = N.to_vec<uint16_t>();
  double eh = 0, en = 0;
  for (size_t r = 0; r < R; ++r) {
    std::vector<double> hv(D);
    double m = 0, v = 0;
    for (size_t c = 0; c < D; ++c) {
      hv[c] = (double)(h2f(proj[r * D + c]) + res[r * D + c]);
      eh = std::max(eh, scaled(h[r * D + c], hv[c]));
      m += hv[c];
    }
    m /= D;
    for (size_t c = 0; c < D; ++c) v += (hv[c] - m) * (hv[c] - m);
    v /= D;
    for (size_t c = 0; c < D; ++c)
      en = std::max(en, scaled(h2f(nn[r * D + c]), (hv[c] - m) / std::sqrt(v + 1e-5) * h2f(w[c])));
  }
  report("triton_residual_add_layernorm h", eh, 1e-6);
  report("triton_residual_add_layernorm y", en, 2e-3);
}

void test_q8_embedding(const RocmDevice& dev, const RocmKernels& k) {
  const size_t vocab = 97, hidden = 416, nb = hidden / 32;
  std::vector<uint8_t> table(vocab * nb * 34);
  for (size_t blk = 0; blk < vocab * nb; ++blk) {
    const uint16_t d = f2h(0.001f + 0.0001f * (float)(blk % 97));
    std::memcpy(&table[blk * 34], &d, 2);
    for (int j = 0; j < 32; ++j) table[blk * 34 + 2 + j] = (uint8_t)(int8_t)((int)((blk * 31 + j * 7) % 255) - 127);
  }
  std::vector<uint32_t> ids = {0, 96, 5, 5, 42, 17, 96, 1};
  QEmbedding emb(dev, k, Tensor::from_host(dev, table.data(), {table.size()}, DType::U8), vocab, hidden);
  Tensor I = Tensor::from_host(dev, ids.data(), {2, 4}, DType::U32);
  Tensor O = emb.forward(I);
  std::vector<float> o = O.to_vec<float>();
  long bad = 0;
  for (size_t n = 0; n < ids.size(); ++n)
    for (size_t j = 0; j < hidden; ++j) {
      const uint8_t* bp = &table[(ids[n] * nb + j / 32) * 34];
      uint16_t d;
      std::memcpy(&d, bp, 2);
      const float ref = (float)(int8_t)bp[2 + j % 32] * h2f(d);  // exact in f32
      if (std::memcmp(&ref, &o[n * hidden + j], 4) != 0) ++bad;
    }
  std::printf("%-34s %ld elements differ (shape [%zu, %zu, %zu]) %s\n", "QEmbedding::forward bit-exact", bad,
              O.dim(0), O.dim(1), O.dim(2), bad == 0 ? "ok" : "FAIL");
  if (bad) ++g_failed;
  std::vector<uint32_t> badids = {3, 97};
  Tensor BI = Tensor::from_host(dev, badids.data(), {2}, DType::U32);
  expect_throw("QEmbedding::forward out of range", [&] { emb.forward(BI); }, "out of range");
}

void test_rotary(const RocmDevice& dev, const RocmKernels& k) {
  const size_t B = 1, Hq = 4, Hk = 2, T = 37, Dh = 64, rot = 32, pos0 = 11;
  RotaryEmbedding re(dev, k, rot, 4096, 10000.0f);
  std::vector<float> q(B * Hq * T * Dh), kk(B * Hk * T * Dh);
  for (size_t i = 0; i < q.size(); ++i) q[i] = std::sin(0.3f * (float)i);
  for (size_t i = 0; i < kk.size(); ++i) kk[i] = std::cos(0.7f * (float)i);
  Tensor Q = Tensor::from_host(dev, q.data(), {B, Hq, T, Dh}, DType::F32);
  Tensor K = Tensor::from_host(dev, kk.data(), {B, Hk, T, Dh}, DType::F32);
  auto [QO, KO] = re.apply(Q, K, pos0);
  dev.synchronize();
  double err = 0;
  auto check = [&](const std::vector<float>& in, const std::vector<float>& out, size_t H) {
    for (size_t h = 0; h < B * H; ++h)
      for (size_t t = 0; t < T; ++t)
        for (size_t i = 0; i < Dh; ++i) {
          const size_t o = (h * T + t) * Dh;
          double ref = in[o + i];
          if (i < rot) {
            const size_t p = i / 2;
            const float inv_freq = 1.0f / std::pow(10000.0f, (2.0f * (float)p) / (float)rot);
            const double ang = (double)((float)(pos0 + t) * inv_freq);
            ref = (i % 2 == 0) ? in[o + i] * std::cos(ang) - in[o + i + 1] * std::sin(ang)
                               : in[o + i] * std::cos(ang) + in[o + i - 1] * std::sin(ang);
          }
          err = std::max(err, scaled(out[o + i], ref));
        }
  };
  check(q, QO.to_vec<float>(), Hq);
  check(kk, KO.to_vec<float>(), Hk);
  report("apply_rotary_pos_emb (RoPE table)", err, 1e-5);
}

// One decoder step after another, as the reference's decoder runs them
// (src/moonshine/gpu_decoder_metal.rs:144-182): RoPE + K cache write, V cache
// append, self-attention over positions 0..pos, then cross-attention over a
// fixed "encoder" K/V with the reference's min(32, kv_len) splits. The
// expected values: float64 rotation (f32 angles as RotaryEmbedding) rounded
// to f16 like the stored q/k, float64 softmax attention.
void test_decode_step(const RocmDevice& dev, const RocmKernels& k) {
  const size_t Hq = 8, Hk = 2, Dh = 64, rot = 32, L = 40, steps = 12, Lx = 70;
  const float scale = 0.125f;
  RotaryEmbedding re(dev, k, rot, L, 10000.0f);
  std::vector<uint16_t> ck(Hk * L * Dh, 0), cv(Hk * L * Dh, 0);  // host mirror of the caches (f16)
  Tensor CK = Tensor::from_host(dev, ck.data(), {Hk, L, Dh}, DType::F16);
  Tensor CV = Tensor::from_host(dev, cv.data(), {Hk, L, Dh}, DType::F16);
  // encoder K/V [Lx, Hk, Dh]
  std::vector<uint16_t> xk(Lx * Hk * Dh), xv(Lx * Hk * Dh);
  for (size_t i = 0; i < xk.size(); ++i) {
    xk[i] = f2h(std::sin(0.011f * (float)i));
    xv[i] = f2h(std::cos(0.017f * (float)i));
  }
  Tensor XK = Tensor::from_host(dev, xk.data(), {Lx, Hk, Dh}, DType::F16);
  Tensor XV = Tensor::from_host(dev, xv.data(), {Lx, Hk, Dh}, DType::F16);
  Tensor partial = Tensor::empty(dev, {Hq * 32 * 384}, DType::F32);
  auto attend = [&](const std::vector<uint16_t>& q, const uint16_t* kk, const uint16_t* vv, size_t n, size_t skh,
                    size_t sks, std::vector<double>& out) {
    for (size_t h = 0; h < Hq; ++h) {
      const size_t kvh = h * Hk / Hq;
      std::vector<double> s(n);
      double m = -1e300;
      for (size_t j = 0; j < n; ++j) {
        double d = 0;
        for (size_t e = 0; e < Dh; ++e) d += (double)h2f(q[h * Dh + e]) * h2f(kk[kvh * skh + j * sks + e]);
        s[j] = d * scale;
        m = std::max(m, s[j]);
      }
      double l = 0;
      for (size_t j = 0; j < n; ++j) l += (s[j] = std::exp(s[j] - m));
      for (size_t e = 0; e < Dh; ++e) {
        double a = 0;
        for (size_t j = 0; j < n; ++j) a += s[j] * h2f(vv[kvh * skh + j * sks + e]);
        out[h * Dh + e] = a / l;
      }
    }
  };
  double err_self = 0, err_cross = 0;
  for (size_t pos = 0; pos < steps; ++pos) {
    std::vector<uint16_t> q(Hq * Dh), kn(Hk * Dh), vn(Hk * Dh);
    for (size_t i = 0; i < q.size(); ++i) q[i] = f2h(std::sin(0.37f * (float)(i + 97 * pos)));
    for (size_t i = 0; i < kn.size(); ++i) kn[i] = f2h(std::cos(0.23f * (float)(i + 53 * pos)));
    for (size_t i = 0; i < vn.size(); ++i) vn[i] = f2h(std::sin(0.13f * (float)(i + 31 * pos)));
    Tensor Q = Tensor::from_host(dev, q.data(), {Hq, Dh}, DType::F16);
    Tensor K = Tensor::from_host(dev, kn.data(), {Hk, Dh}, DType::F16);
    Tensor V = Tensor::from_host(dev, vn.data(), {Hk, Dh}, DType::F16);
    Tensor O = Tensor::empty(dev, {Hq, Dh}, DType::F16);
    Tensor OX = Tensor::empty(dev, {Hq, Dh}, DType::F16);
    enc_rope_qk_cache_fused(dev.stream(), k, Q.buffer(), K.buffer(), re.table().buffer(), CK.buffer(), pos, L, Hq,
                            Hk, Dh, rot);
    if (pos % 2 == 0) {  // buffer-level and tensor-level forms on alternate steps
      enc_kv_cache_append(dev.stream(), k, V.buffer(), CV.buffer(), Hk, Dh, L, pos);
      enc_attention_decode(dev.stream(), k, Q.buffer(), CK.buffer(), CV.buffer(), O.buffer(), pos + 1, Dh, Hk, Hq,
                           scale, L * Dh, Dh);
    } else {
      triton_kv_cache_append(dev, k, V, CV, Hk, Dh, L, pos);
      triton_attention_decode(dev, k, Q, CK, CV, O, pos + 1, Dh, Hk, Hq, scale, L * Dh, Dh);
    }
    const size_t splits = std::min<size_t>(32, Lx);
    enc_attention_splitkv(dev.stream(), k, Q.buffer(), XK.buffer(), XV.buffer(), OX.buffer(), partial.buffer(), Lx,
                          Dh, Hk, Hq, scale, Dh, Hk * Dh, splits);
    dev.synchronize();
    // host: rotate q, k (f32 angle, float64 products, f16 store), append to the caches
    auto rope = [&](std::vector<uint16_t>& x, size_t H) {
      for (size_t h = 0; h < H; ++h)
        for (size_t p = 0; p < rot / 2; ++p) {
          const float inv_freq = 1.0f / std::pow(10000.0f, (2.0f * (float)p) / (float)rot);
          const double ang = (double)((float)pos * inv_freq);
          const double x0 = h2f(x[h * Dh + 2 * p]), x1 = h2f(x[h * Dh + 2 * p + 1]);
          x[h * Dh + 2 * p] = f2h((float)(x0 * std::cos(ang) - x1 * std::sin(ang)));
          x[h * Dh + 2 * p + 1] = f2h((float)(x1 * std::cos(ang) + x0 * std::sin(ang)));
        }
    };
    rope(q, Hq);
    rope(kn, Hk);
    for (size_t h = 0; h < Hk; ++h)
      for (size_t e = 0; e < Dh; ++e) {
        ck[(h * L + pos) * Dh + e] = kn[h * Dh + e];
        cv[(h * L + pos) * Dh + e] = vn[h * Dh + e];
      }
    std::vector<double> ref(Hq * Dh), refx(Hq * Dh);
    attend(q, ck.data(), cv.data(), pos + 1, L * Dh, Dh, ref);
    attend(q, xk.data(), xv.data(), Lx, Dh, Hk * Dh, refx);
    const std::vector<uint16_t> o = O.to_vec<uint16_t>(), ox = OX.to_vec<uint16_t>();
    for (size_t i = 0; i < ref.size(); ++i) {
      err_self = std::max(err_self, scaled(h2f(o[i]), ref[i]));
      err_cross = std::max(err_cross, scaled(h2f(ox[i]), refx[i]));
    }
  }
  report("decode step: rope+cache, self-attn", err_self, 2e-3);
  report("decode step: cross-attn (splitkv)", err_cross, 2e-3);
}

void test_errors(const RocmDevice& dev, const RocmKernels& k) {
  float host[8] = {0};
  Tensor C = Tensor::cpu(host, {2, 4}, DType::F32);
  Tensor D = Tensor::empty(dev, {2, 4}, DType::F16);
  expect_throw("host tensor is rejected", [&] { triton_layernorm_std_f32in(dev, k, C, D, D, 2, 4); },
               "must be on the ROCm device");
  Tensor X = Tensor::empty(dev, {2, 4}, DType::F16);
  expect_throw("wrong dtype is rejected", [&] { triton_layernorm_std_f32in(dev, k, X, D, D, 2, 4); },
               "expected f32");
  Tensor Xf = Tensor::empty(dev, {2, 4}, DType::F32);
  expect_throw("short tensor is rejected", [&] { triton_layernorm_std_f32in(dev, k, Xf, D, D, 4, 4); },
               "need 16");
  Tensor Q = Tensor::empty(dev, {2, 64}, DType::F16);
  Tensor Kc = Tensor::empty(dev, {2, 10, 64}, DType::F16);
  expect_throw("attention over more positions than the cache holds is rejected",
               [&] { triton_attention_decode(dev, k, Q, Kc, Kc, Q, 11, 64, 2, 2, 0.125f, 640, 64); }, "need");
  RocmKokoroBackend be(dev, k);
  expect_throw("adain_snake f16 row past the limit is rejected",
               [&] { be.adain_snake(X.buffer(), X.buffer(), X.buffer(), X.buffer(), X.buffer(), 1, 200000); },
               "131072");
}

// The same self-test inputs through the f16-activation form: x rounded to
// f16, the f64 expectation taken on the rounded input, f16 output (2e-3 of
// max(|ref|, 1), an f16 ulp being at most 9.8e-4 of the value).
void test_adain_snake_f16(const RocmDevice& dev, const RocmKernels& k, size_t C, size_t T, const char* name) {
  std::vector<uint16_t> x(C * T);
  for (size_t i = 0; i < x.size(); ++i) x[i] = f2h(std::sin(0.001f * (float)i) * 3.0f);
  std::vector<uint16_t> g(C), b(C), a(C);
  for (size_t c = 0; c < C; ++c) {
    g[c] = f2h(std::sin(0.01f * (float)c) * 0.5f);
    b[c] = f2h(std::cos(0.02f * (float)c) * 0.3f);
    a[c] = f2h(1.0f + std::sin(0.005f * (float)c));
  }
  Tensor X = Tensor::from_host(dev, x.data(), {C, T}, DType::F16);
  Tensor G = Tensor::from_host(dev, g.data(), {C}, DType::F16);
  Tensor B = Tensor::from_host(dev, b.data(), {C}, DType::F16);
  Tensor A = Tensor::from_host(dev, a.data(), {C}, DType::F16);
  Tensor O = Tensor::empty(dev, {C, T}, DType::F16);
  RocmKokoroBackend be(dev, k);
  be.adain_snake(X.buffer(), G.buffer(), B.buffer(), A.buffer(), O.buffer(), C, T);
  dev.synchronize();
  std::vector<uint16_t> o = O.to_vec<uint16_t>();
  double err = 0;
  for (size_t c = 0; c < C; ++c) {
    double mean = 0, var = 0;
    for (size_t t = 0; t < T; ++t) mean += h2f(x[c * T + t]);
    mean /= (double)T;
    for (size_t t = 0; t < T; ++t) var += (h2f(x[c * T + t]) - mean) * (h2f(x[c * T + t]) - mean);
    var /= (double)T;
    const double al = h2f(a[c]);
    const double inv_a = (double)(1.0f / (h2f(a[c]) + 1e-9f));
    for (size_t t = 0; t < T; ++t) {
      const double y = (h2f(x[c * T + t]) - mean) / std::sqrt(var + 1e-5) * (1.0 + h2f(g[c])) + h2f(b[c]);
      const double s = std::sin(al * y);
      err = std::max(err, scaled(h2f(o[c * T + t]), y + s * s * inv_a));
    }
  }
  report(name, err, 2e-3);
}

// snake alone (gpu_backend.rs:51-52) on the same inputs, f16 in and out.
void test_snake_f16(const RocmDevice& dev, const RocmKernels& k, size_t C, size_t T) {
  std::vector<uint16_t> x(C * T), a(C);
  for (size_t i = 0; i < x.size(); ++i) x[i] = f2h(std::sin(0.001f * (float)i) * 3.0f);
  for (size_t c = 0; c < C; ++c) a[c] = f2h(1.0f + std::sin(0.005f * (float)c));
  Tensor X = Tensor::from_host(dev, x.data(), {C, T}, DType::F16);
  Tensor A = Tensor::from_host(dev, a.data(), {C}, DType::F16);
  Tensor O = Tensor::empty(dev, {C, T}, DType::F16);
  RocmKokoroBackend be(dev, k);
  be.snake(X.buffer(), A.buffer(), O.buffer(), C * T, C, T);
  dev.synchronize();
  std::vector<uint16_t> o = O.to_vec<uint16_t>();
  double err = 0;
  for (size_t c = 0; c < C; ++c)
    for (size_t t = 0; t < T; ++t) {
      const double v = h2f(x[c * T + t]), al = h2f(a[c]);
      const double s = std::sin(al * v);
      err = std::max(err, scaled(h2f(o[c * T + t]), v + s * s / (al + 1e-9)));
    }
  report("snake (f16) C=16 T=3001", err, 2e-3);
}

// The generator tail through the backend methods, the reference's order
// (decoder.rs:542-589): add_f32 twice, scale_third_f32, leaky_relu_f32 (bit-
// exact against the same f32 operations on the host), conv1d_f32 into 22
// channels (float64 host conv, 1e-5 of max(|ref|, 1)) and istft_gpu (float64
// host overlap-add of the same formulas, 1e-5 of max(|ref|, 1)).
void test_kokoro_tail(const RocmDevice& dev, const RocmKernels& k) {
  const size_t C = 32, T = 301, n = C * T, CO = 22, K = 7;
  std::vector<float> r0(n), r1(n), r2(n);
  for (size_t i = 0; i < n; ++i) {
    r0[i] = std::sin(0.013f * (float)i);
    r1[i] = std::cos(0.007f * (float)i) * 0.5f;
    r2[i] = std::sin(0.031f * (float)i + 1.0f) * 0.8f;
  }
  Tensor R0 = Tensor::from_host(dev, r0.data(), {C, T}, DType::F32);
  Tensor R1 = Tensor::from_host(dev, r1.data(), {C, T}, DType::F32);
  Tensor R2 = Tensor::from_host(dev, r2.data(), {C, T}, DType::F32);
  Tensor S = Tensor::empty(dev, {C, T}, DType::F32), S2 = Tensor::empty(dev, {C, T}, DType::F32);
  Tensor A = Tensor::empty(dev, {C, T}, DType::F32), L = Tensor::empty(dev, {C, T}, DType::F32);
  RocmKokoroBackend be(dev, k);
  be.add_f32(R0.buffer(), R1.buffer(), S.buffer(), n);
  be.add_f32(S.buffer(), R2.buffer(), S2.buffer(), n);
  be.scale_third_f32(S2.buffer(), A.buffer(), n);
  be.leaky_relu_f32(A.buffer(), L.buffer(), n, 0.01f);
  // conv_post: 32 -> 22 channels, K = 7, padding 3
  std::vector<uint16_t> w(CO * C * K), b(CO);
  for (size_t i = 0; i < w.size(); ++i) w[i] = f2h(0.05f * std::cos(0.37f * (float)i));
  for (size_t i = 0; i < CO; ++i) b[i] = f2h(-0.5f + 0.01f * (float)i);
  Tensor W = Tensor::from_host(dev, w.data(), {CO, C, K}, DType::F16);
  Tensor Bi = Tensor::from_host(dev, b.data(), {CO}, DType::F16);
  Tensor X = Tensor::empty(dev, {CO, T}, DType::F32);
  be.conv1d_f32(L.buffer(), W.buffer(), Bi.buffer(), X.buffer(), C, CO, T, T, K, 1, 3, 1);
  const size_t out_len = (T - 1) * 5;
  Tensor AU = Tensor::empty(dev, {out_len}, DType::F32);
  be.istft_gpu(X.buffer(), AU.buffer(), T, out_len);
  dev.synchronize();
  // host: the same f32 element-wise chain
  std::vector<float> lr(n);
  bool exact = true;
  const std::vector<float> l_gpu = L.to_vec<float>();
  for (size_t i = 0; i < n; ++i) {
    float v = (r0[i] + r1[i]) + r2[i];
    v = v * (float)0.3333333333333333;
    v = v > 0.f ? v : v * 0.01f;
    lr[i] = v;
    if (std::memcmp(&v, &l_gpu[i], 4) != 0) exact = false;
  }
  report("tail: add, add, scale_third, leaky_relu bit-exact", exact ? 0.0 : 1.0, 0.0);
  // host conv in float64 on the GPU's own leaky-ReLU output
  std::vector<double> xr(CO * T, 0.0);
  for (size_t o = 0; o < CO; ++o)
    for (size_t t = 0; t < T; ++t) {
      double acc = h2f(b[o]);
      for (size_t c = 0; c < C; ++c)
        for (size_t kk = 0; kk < K; ++kk) {
          const long ti = (long)t + (long)kk - 3;
          if (ti >= 0 && ti < (long)T) acc += (double)h2f(w[(o * C + c) * K + kk]) * l_gpu[c * T + (size_t)ti];
        }
      xr[o * T + t] = acc;
    }
  const std::vector<float> x_gpu = X.to_vec<float>();
  double err = 0;
  for (size_t i = 0; i < xr.size(); ++i) err = std::max(err, scaled(x_gpu[i], xr[i]));
  report("tail: conv1d_f32 (conv_post)", err, 1e-5);
  // host iSTFT in float64 on the GPU's conv output
  const int N = 20, hop = 5, bins = 11;
  const double PI = 3.14159265358979323846;
  std::vector<double> y((T - 1) * hop + N, 0.0), ws(y.size(), 0.0);
  for (size_t f = 0; f < T; ++f)
    for (int nn = 0; nn < N; ++nn) {
      double v = 0;
      for (int kb = 0; kb < bins; ++kb) {
        const double m = std::exp((double)x_gpu[kb * T + f]), p = std::sin((double)x_gpu[(bins + kb) * T + f]);
        const double sc = (kb == 0 || kb == bins - 1) ? 1.0 : 2.0;
        const double ang = 2 * PI * kb * nn / N;
        v += sc * (m * std::cos(p) * std::cos(ang) - m * std::sin(p) * std::sin(ang));
      }
      const double wn = 0.5 - 0.5 * std::cos(2 * PI * nn / N);
      y[f * hop + nn] += v / N * wn;
      ws[f * hop + nn] += wn * wn;
    }
  const std::vector<float> au = AU.to_vec<float>();
  double err2 = 0;
  for (size_t i = 0; i < out_len; ++i) {
    const size_t pp = i + N / 2;
    const double ref = ws[pp] > 1e-8 ? y[pp] / ws[pp] : 0.0;
    err2 = std::max(err2, scaled(au[i], ref));
  }
  report("tail: istft_gpu", err2, 1e-5);
}

// The decoder MLP GEMVs through the buffer-level mirror: fc1 + bias + GLU and
// fc2 + residual + LN at a small Moonshine-like shape, against float64 host
// sums of the dequantised weights (f16 outputs: 2e-3 of max(|ref|, 1)).
void test_gemv_q8(const RocmDevice& dev, const RocmKernels& k) {
  const size_t K = 96, N = 64;  // fc1: K -> 2N (GLU to N); fc2: N -> K
  std::vector<uint16_t> x(K), x2(N);
  for (size_t i = 0; i < K; ++i) x[i] = f2h(std::sin(0.3f * (float)i));
  std::vector<uint32_t> qs1(K * 2 * N / 4), qs2(N * K / 4);
  std::vector<uint16_t> sc1(K / 32 * 2 * N), sc2(N / 32 * K), lnw(K);
  uint32_t st = 12345u;
  auto rnd = [&]() { st = st * 1664525u + 1013904223u; return st; };
  for (auto& w : qs1) w = rnd();
  for (auto& w : qs2) w = rnd();
  for (size_t i = 0; i < sc1.size(); ++i) sc1[i] = f2h(0.002f * (1 + (float)(i % 7)));
  for (size_t i = 0; i < sc2.size(); ++i) sc2[i] = f2h(0.002f * (1 + (float)(i % 5)));
  for (size_t i = 0; i < K; ++i) lnw[i] = f2h(1.0f + 0.01f * (float)(i % 9));
  std::vector<float> bias(2 * N), res(K);
  for (size_t i = 0; i < 2 * N; ++i) bias[i] = 0.1f * std::cos((float)i);
  for (size_t i = 0; i < K; ++i) res[i] = std::sin(0.11f * (float)i);
  auto wq = [](const std::vector<uint32_t>& qs, const std::vector<uint16_t>& sc, size_t NW, size_t kk, size_t j) {
    const int8_t q = (int8_t)((qs[kk * (NW / 4) + j / 4] >> (8 * (j % 4))) & 0xff);
    return (double)q * h2f(sc[(kk / 32) * NW + j]);
  };
  Tensor X = Tensor::from_host(dev, x.data(), {K}, DType::F16);
  Tensor Q1 = Tensor::from_host(dev, qs1.data(), {qs1.size()}, DType::U32);
  Tensor S1 = Tensor::from_host(dev, sc1.data(), {sc1.size()}, DType::F16);
  Tensor B1 = Tensor::from_host(dev, bias.data(), {2 * N}, DType::F32);
  Tensor H = Tensor::empty(dev, {N}, DType::F16);
  enc_gemv_q8_bias_glu(dev.stream(), k, X.buffer(), Q1.buffer(), S1.buffer(), B1.buffer(), H.buffer(), K, N);
  dev.synchronize();
  const std::vector<uint16_t> h = H.to_vec<uint16_t>();
  double err = 0;
  for (size_t j = 0; j < N; ++j) {
    double up = bias[j], gate = bias[N + j];
    for (size_t kk = 0; kk < K; ++kk) {
      up += (double)h2f(x[kk]) * wq(qs1, sc1, 2 * N, kk, j);
      gate += (double)h2f(x[kk]) * wq(qs1, sc1, 2 * N, kk, N + j);
    }
    err = std::max(err, scaled(h2f(h[j]), gate / (1 + std::exp(-gate)) * up));
  }
  report("enc_gemv_q8_bias_glu", err, 2e-3);
  // the mirror packs the weight to t4 tiles on its first call and reuses the copy: a second call adds no
  // cache entry and gives the same bits
  if (k.gemv_weights_cached() != 1) throw Error("enc_gemv_q8_bias_glu: expected one cached t4 weight");
  enc_gemv_q8_bias_glu(dev.stream(), k, X.buffer(), Q1.buffer(), S1.buffer(), B1.buffer(), H.buffer(), K, N);
  dev.synchronize();
  if (H.to_vec<uint16_t>() != h || k.gemv_weights_cached() != 1)
    throw Error("enc_gemv_q8_bias_glu: second call differs or packed again");
  // the plain GEMV over the x half of the same buffers (NW = N columns of a [K, N/4] weight): its own cache entry
  {
    std::vector<uint32_t> qp(K * N / 4);
    std::vector<uint16_t> sp(K / 32 * N);
    for (size_t kk = 0; kk < K; ++kk)
      for (size_t j = 0; j < N / 4; ++j) qp[kk * (N / 4) + j] = qs1[kk * (2 * N / 4) + j];
    for (size_t b = 0; b < K / 32; ++b)
      for (size_t j = 0; j < N; ++j) sp[b * N + j] = sc1[b * 2 * N + j];
    Tensor QP = Tensor::from_host(dev, qp.data(), {qp.size()}, DType::U32);
    Tensor SP = Tensor::from_host(dev, sp.data(), {sp.size()}, DType::F16);
    Tensor OP = Tensor::empty(dev, {N}, DType::F16);
    enc_gemv_q8(dev.stream(), k, X.buffer(), QP.buffer(), SP.buffer(), nullptr, OP.buffer(), K, N);
    dev.synchronize();
    const std::vector<uint16_t> op = OP.to_vec<uint16_t>();
    double e = 0;
    for (size_t j = 0; j < N; ++j) {
      double up = 0;
      for (size_t kk = 0; kk < K; ++kk) up += (double)h2f(x[kk]) * wq(qp, sp, N, kk, j);
      e = std::max(e, scaled(h2f(op[j]), up));
    }
    report("enc_gemv_q8 (t4 copy)", e, 2e-3);
    if (k.gemv_weights_cached() != 2) throw Error("enc_gemv_q8: expected a second cached t4 weight");
  }
  Tensor Q2 = Tensor::from_host(dev, qs2.data(), {qs2.size()}, DType::U32);
  Tensor S2 = Tensor::from_host(dev, sc2.data(), {sc2.size()}, DType::F16);
  Tensor RS = Tensor::from_host(dev, res.data(), {K}, DType::F32);
  Tensor LW = Tensor::from_host(dev, lnw.data(), {K}, DType::F16);
  Tensor OF = Tensor::empty(dev, {K}, DType::F32);
  Tensor NM = Tensor::empty(dev, {K}, DType::F16);
  enc_gemv_q8_resadd_ln(dev.stream(), k, H.buffer(), Q2.buffer(), S2.buffer(), RS.buffer(), OF.buffer(), LW.buffer(),
                        NM.buffer(), N, K, 1e-5f);
  dev.synchronize();
  const std::vector<float> of = OF.to_vec<float>();
  const std::vector<uint16_t> nm = NM.to_vec<uint16_t>();
  std::vector<double> hv(K);
  double err_h = 0, mean = 0, var = 0;
  for (size_t j = 0; j < K; ++j) {
    double acc = 0;
    for (size_t kk = 0; kk < N; ++kk) acc += (double)h2f(h[kk]) * wq(qs2, sc2, K, kk, j);
    hv[j] = (double)h2f(f2h((float)acc)) + res[j];
    err_h = std::max(err_h, scaled(of[j], hv[j]));
    mean += hv[j];
  }
  mean /= (double)K;
  for (size_t j = 0; j < K; ++j) var += (hv[j] - mean) * (hv[j] - mean);
  var /= (double)K;
  double err_n = 0;
  for (size_t j = 0; j < K; ++j)
    err_n = std::max(err_n, scaled(h2f(nm[j]), (hv[j] - mean) / std::sqrt(var + 1e-5) * h2f(lnw[j])));
  report("enc_gemv_q8_resadd_ln h", err_h, 2e-3);
  report("enc_gemv_q8_resadd_ln norm", err_n, 2e-3);
  if (k.gemv_weights_cached() != 3) throw Error("enc_gemv_q8_resadd_ln: expected a third cached t4 weight");
  k.forget_gemv_weights();
  if (k.gemv_weights_cached() != 0) throw Error("forget_gemv_weights left entries");
}

}  // namespace

int main() {
  try {
    RocmDevice dev = RocmDevice::create(0);
    RocmKernels k = RocmKernels::load(dev);
    std::printf("kernels loaded: %d probed\n", k.kernel_count());
    test_adain_snake_f32(dev, k, 4, 100, "adain_snake_f32 C=4 T=100");
    test_adain_snake_f32(dev, k, 128, 11281, "adain_snake_f32 C=128 T=11281");
    test_adain_snake_f16(dev, k, 4, 100, "adain_snake (f16) C=4 T=100");
    test_adain_snake_f16(dev, k, 128, 11281, "adain_snake (f16) C=128 T=11281");
    test_snake_f16(dev, k, 16, 3001);
    test_kokoro_tail(dev, k);
    test_gemv_q8(dev, k);
    test_layernorm_std_f32in(dev, k);
    test_layernorm_unit_offset_and_bare(dev, k);
    test_elementwise(dev, k);
    test_residual_add_layernorm(dev, k);
    test_q8_embedding(dev, k);
    test_rotary(dev, k);
    test_decode_step(dev, k);
    test_errors(dev, k);
  } catch (const Error& e) {
    std::printf("unexpected error: %s\n", e.what());
    return 2;
  }
  std::printf("%s: %d failed\n", g_failed ? "FAILED" : "PASSED", g_failed);
  return g_failed ? 1 : 0;
}
