// Synthetic benchmark inputs (measurement support, host code): the seeded
// generator the benchmark configurations are specified with.
//
// One stream per tensor: xoshiro256** (Blackman and Vigna, 2018) whose 256-bit
// state is filled by splitmix64 from the 64-bit seed 24301 ^ fnv1a64(name)
// (24301: the reference workload's seed, agent/workload.toml:2; name: e.g.
// "2/x" for tensor x of configuration 2).  Uniform doubles are the top 53 bits
// of an output times 2^-53.  Normals come in pairs from Box-Muller in double
// (r = sqrt(-2 ln(1 - u1)), angle 2 pi u2), are scaled to mean + std * z in
// double, rounded to f32, and for bf16 outputs rounded to bf16 (nearest even).
// Outliers (probability p per element, p > 0): a second stream, seeded from
// name + "#bernoulli", draws one uniform per element and selects it when the
// uniform is below p; the selected element becomes outlier_x * z' with z' from
// a third stream (name + "#outlier") drawn in selection order.
#include <cmath>
#include <cstring>

#include "k3h_internal.h"

namespace {

constexpr uint64_t kSeedBase = 24301;

uint64_t fnv1a64(const char* s) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (; *s; ++s) {
    h ^= (unsigned char)*s;
    h *= 0x100000001b3ull;
  }
  return h;
}

uint64_t splitmix64(uint64_t* x) {
  uint64_t z = (*x += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

struct Xoshiro {
  uint64_t s[4];
  explicit Xoshiro(uint64_t seed) {
    for (auto& w : s) w = splitmix64(&seed);
  }
  static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
  uint64_t next() {
    const uint64_t r = rotl(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return r;
  }
  double uniform() { return (double)(next() >> 11) * 0x1.0p-53; }
};

// Box-Muller pairs, handed out one at a time.
struct Normal {
  Xoshiro x;
  double spare = 0.0;
  bool have = false;
  explicit Normal(uint64_t seed) : x(seed) {}
  double next() {
    if (have) {
      have = false;
      return spare;
    }
    const double u1 = x.uniform(), u2 = x.uniform();
    const double r = std::sqrt(-2.0 * std::log(1.0 - u1));
    const double a = 6.283185307179586476925 * u2;
    spare = r * std::sin(a);
    have = true;
    return r * std::cos(a);
  }
};

uint16_t bf16_rne(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // NaN stays NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

uint64_t seed_of(const char* name, const char* suffix) {
  char buf[256];
  std::strncpy(buf, name, sizeof(buf) - 16);
  buf[sizeof(buf) - 16] = 0;
  std::strcat(buf, suffix);
  return kSeedBase ^ fnv1a64(buf);
}

}  // namespace

extern "C" {

K3H_API int k3h_synth_normal(const char* name, size_t n, float mean, float std_dev, float outlier_p,
                             float outlier_x, int bf16_out, void* out) {
  if (!name || !out || !(std_dev >= 0.0f) || !(outlier_p >= 0.0f && outlier_p <= 1.0f) ||
      std::strlen(name) > 200)
    return K3H_EINVAL;
  Normal g(seed_of(name, ""));
  Xoshiro pick(seed_of(name, "#bernoulli"));
  Normal big(seed_of(name, "#outlier"));
  uint16_t* o16 = static_cast<uint16_t*>(out);
  float* o32 = static_cast<float*>(out);
  for (size_t i = 0; i < n; ++i) {
    double v = (double)mean + (double)std_dev * g.next();
    if (outlier_p > 0.0f && pick.uniform() < (double)outlier_p) v = (double)outlier_x * big.next();
    const float f = (float)v;
    if (bf16_out) o16[i] = bf16_rne(f);
    else o32[i] = f;
  }
  return K3H_OK;
}

}  // extern "C"
