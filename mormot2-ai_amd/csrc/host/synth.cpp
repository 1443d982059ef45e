// synth.cpp - seeded synthetic weights in every block type, written on the
// host (the random generators of the reference's tests,
// tests/test.infer.fast.pas:144-260, generalised): rows are generated
// independently from splitmix64 streams, so any thread count writes the same
// bytes.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <thread>

#include "internal.h"

namespace ihip {

struct Rng {
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed) {}
  // splitmix64 (the generator of sampler.pas:8-12 in the reference)
  uint64_t next()
  {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  double uniform() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }
  double normal()
  {
    double u1 = uniform(), u2 = uniform();
    if (u1 < 1e-300) u1 = 1e-300;
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(2 * M_PI * u2);
  }
};

static inline uint16_t f2h(float f)
{
  // IEEE single -> half, round to nearest even (subnormals, overflow to inf)
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u, mant = x & 0x7fffffu;
  int exp = (int)((x >> 23) & 0xff);
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u | (mant >> 13) : 0u));
  exp = exp - 127 + 15;
  if (exp >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (exp <= 0) {
    if (exp < -10) return (uint16_t)sign;
    mant |= 0x800000u;
    uint32_t shift = (uint32_t)(14 - exp), h = mant >> shift, rem = mant & ((1u << shift) - 1),
             halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (h & 1))) h++;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)exp << 10) | (mant >> 13), rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
  return (uint16_t)(sign | h);
}

static inline uint16_t f2bf(float f)
{
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fff + ((u >> 16) & 1);
  return (uint16_t)(u >> 16);
}

static uint64_t row_seed(uint64_t seed, int64_t r)
{
  Rng g(seed ^ (0xA0761D6478BD642Full * (uint64_t)(r + 1)));
  return g.next();
}

static void run_rows(int64_t rows, int threads, const std::function<void(int64_t)>& fn)
{
  unsigned nt = threads > 0 ? (unsigned)threads : std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (nt <= 1 || rows < 64) {
    for (int64_t r = 0; r < rows; r++) fn(r);
    return;
  }
  std::vector<std::thread> th;
  for (unsigned t = 0; t < nt; t++)
    th.emplace_back([&, t] {
      for (int64_t r = t; r < rows; r += nt) fn(r);
    });
  for (auto& x : th) x.join();
}

static float scale_in(Rng& g, int lo, int hi)
{
  double a = std::ldexp(1.0, lo), b = std::ldexp(1.0, hi);
  return (float)(a + (b - a) * g.uniform());
}

// codes uniform, scales uniform in [2^lo, 2^hi]
static void blocks_row(uint8_t* r, int t, int64_t cols, Rng& g, int lo, int hi)
{
  const int64_t nb = cols / block_values(t);
  for (int64_t b = 0; b < nb; b++) {
    switch (t) {
    case DT_Q8_0: {
      uint8_t* p = r + b * 34;
      uint16_t d = f2h(scale_in(g, lo, hi));
      memcpy(p, &d, 2);
      for (int j = 0; j < 32; j++) p[2 + j] = (uint8_t)(g.next() & 255);
      break;
    }
    case DT_Q4_0: case DT_Q5_0: case DT_Q5_1: {
      int bs = block_bytes(t);
      uint8_t* p = r + b * bs;
      for (int j = 0; j < bs; j++) p[j] = (uint8_t)(g.next() & 255);
      uint16_t d = f2h(scale_in(g, lo, hi));
      memcpy(p, &d, 2);
      if (t == DT_Q5_1) {
        uint16_t m = f2h(-scale_in(g, lo, hi) * 16.0f);
        memcpy(p + 2, &m, 2);
      }
      break;
    }
    case DT_MXFP4: {
      uint8_t* p = r + b * 17;
      // 2^(e - 127) in [2^lo, 2^hi]
      int e0 = 127 + lo, e1 = 127 + hi;
      p[0] = (uint8_t)(e0 + (int)(g.next() % (uint64_t)(e1 - e0 + 1)));
      for (int j = 0; j < 16; j++) p[1 + j] = (uint8_t)(g.next() & 255);
      break;
    }
    case DT_Q4_K: {
      uint8_t* p = r + b * 144;
      for (int j = 0; j < 144; j++) p[j] = (uint8_t)(g.next() & 255);
      uint16_t d = f2h(scale_in(g, lo, hi)), dm = f2h(scale_in(g, lo, hi));
      memcpy(p, &d, 2);
      memcpy(p + 2, &dm, 2);
      break;
    }
    case DT_Q6_K: {
      uint8_t* p = r + b * 210;
      for (int j = 0; j < 208; j++) p[j] = (uint8_t)(g.next() & 255);
      uint16_t d = f2h(scale_in(g, lo, hi));
      memcpy(p + 208, &d, 2);
      break;
    }
    }
  }
}

static int round_away(float t)
{
  float a = std::fabs(t);
  int f = (int)a;
  if (a - (float)f >= 0.5f) f++;
  return t < 0 ? -f : f;
}

// ~N(0, sigma) weights of row r
static void normal_row(uint8_t* r, int t, int64_t cols, Rng& g, float sigma)
{
  if (t == DT_F32 || t == DT_BF16 || t == DT_F16 || t == DT_Q8_0 || t == DT_Q4_0) {
    std::vector<float> v(cols);
    for (auto& x : v) x = (float)(g.normal() * sigma);
    if (t == DT_F32) {
      memcpy(r, v.data(), cols * 4);
    } else if (t == DT_BF16) {
      for (int64_t i = 0; i < cols; i++) {
        uint16_t u = f2bf(v[i]);
        memcpy(r + 2 * i, &u, 2);
      }
    } else if (t == DT_F16) {
      for (int64_t i = 0; i < cols; i++) {
        uint16_t u = f2h(v[i]);
        memcpy(r + 2 * i, &u, 2);
      }
    } else if (t == DT_Q8_0) {
      // the GGUF writers' ties-away Q8_0 (quantize_row_q8_0_ref,
      // backend.cpu.pas:692-696)
      for (int64_t b = 0; b < cols / 32; b++) {
        float amax = 0;
        for (int j = 0; j < 32; j++) amax = std::max(amax, std::fabs(v[b * 32 + j]));
        float d = amax / 127.0f;
        uint16_t h = f2h(d);
        uint8_t* p = r + b * 34;
        memcpy(p, &h, 2);
        float id = d != 0 ? 1.0f / d : 0.0f;
        for (int j = 0; j < 32; j++) p[2 + j] = (uint8_t)(int8_t)round_away(v[b * 32 + j] * id);
      }
    } else {
      // Q4_0 (InferQuantizeRowQ4_0, backend.cpu.pas:703-756)
      for (int64_t b = 0; b < cols / 32; b++) {
        float amax = 0, m = 0;
        for (int j = 0; j < 32; j++)
          if (amax < std::fabs(v[b * 32 + j])) {
            amax = std::fabs(v[b * 32 + j]);
            m = v[b * 32 + j];
          }
        float d = m / -8.0f;
        uint16_t h = f2h(d);
        uint8_t* p = r + b * 18;
        memcpy(p, &h, 2);
        float id = d != 0 ? 1.0f / d : 0.0f;
        for (int j = 0; j < 16; j++) {
          int q0 = std::min(15, (int)((float)((double)v[b * 32 + j] * id + 8.5)));
          int q1 = std::min(15, (int)((float)((double)v[b * 32 + 16 + j] * id + 8.5)));
          p[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
      }
    }
    return;
  }
  const int64_t nb = cols / block_values(t);
  for (int64_t b = 0; b < nb; b++) {
    switch (t) {
    case DT_Q4_K: {
      // q uniform 0..15 (sd 4.61), value = d sc q - dmin m with dmin = 8 d and
      // m = round(7.5 sc / 8): mean ~0, sd ~ d sc 4.61
      uint8_t* p = r + b * 144;
      float d = sigma / (4.61f * 51.5f);
      uint16_t hd = f2h(d), hm = f2h(8.0f * d);
      memcpy(p, &hd, 2);
      memcpy(p + 2, &hm, 2);
      int sc[8], mn[8];
      for (int j = 0; j < 8; j++) {
        sc[j] = 40 + (int)(g.next() % 24);
        mn[j] = std::min(63, (int)std::lround(sc[j] * 7.5 / 8.0));
      }
      uint8_t* s = p + 4;
      memset(s, 0, 12);
      for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
      }
      for (int j = 0; j < 128; j++) p[16 + j] = (uint8_t)(g.next() & 255);
      break;
    }
    case DT_Q6_K: {
      // q - 32 uniform -32..31 (sd 18.5), positive int8 scales 16..127
      uint8_t* p = r + b * 210;
      for (int j = 0; j < 192; j++) p[j] = (uint8_t)(g.next() & 255);
      for (int j = 0; j < 16; j++) p[192 + j] = (uint8_t)(16 + g.next() % 112);
      uint16_t hd = f2h(sigma / (18.5f * 71.5f));
      memcpy(p + 208, &hd, 2);
      break;
    }
    case DT_MXFP4: {
      // doubled e2m1 codes (sd 5.85) times 2^(e - 128), e around the spread
      uint8_t* p = r + b * 17;
      int e = 128 + (int)std::lround(std::log2(sigma / 5.85));
      p[0] = (uint8_t)std::min(143, std::max(104, e - 1 + (int)(g.next() % 3)));
      for (int j = 0; j < 16; j++) p[1 + j] = (uint8_t)(g.next() & 255);
      break;
    }
    default:
      blocks_row(r + b * block_bytes(t), t, block_values(t), g, -8, -4);
      break;
    }
  }
}

}  // namespace ihip

using namespace ihip;

extern "C" {

int ihip_synth_blocks(void* dst, int t, int64_t rows, int64_t cols, uint64_t seed, int lo, int hi,
                      int threads)
{
  if (!dst || rows < 1 || !block_values(t) || cols % block_values(t) || t == DT_F32 ||
      t == DT_BF16 || t == DT_F16 || lo > hi)
    return fail(IHIP_E_ARG, "ihip_synth_blocks");
  const uint64_t rb = row_bytes(t, cols);
  run_rows(rows, threads, [&](int64_t r) {
    Rng g(row_seed(seed, r));
    blocks_row((uint8_t*)dst + r * rb, t, cols, g, lo, hi);
  });
  return 0;
}

int ihip_synth_normal(void* dst, int t, int64_t rows, int64_t cols, uint64_t seed, float sigma,
                      int threads)
{
  if (!dst || rows < 1 || !block_values(t) || cols % block_values(t) || !(sigma > 0))
    return fail(IHIP_E_ARG, "ihip_synth_normal");
  const uint64_t rb = row_bytes(t, cols);
  run_rows(rows, threads, [&](int64_t r) {
    Rng g(row_seed(seed, r));
    normal_row((uint8_t*)dst + r * rb, t, cols, g, sigma);
  });
  return 0;
}

}  // extern "C"
