// gf256.cpp — host GF(2^8) algebra and the host entry points of the C ABI
// (ec_gf_mul, ec_gf_inv, ec_cauchy_matrix, ec_gf_invert, ec_decode_matrix,
// ec_abi_version, ec_strerror).
//
// Products use log/antilog tables of the generator 0x02 (a primitive element
// for 0x11D: its powers run through all 255 non-zero bytes).  The tables are
// built once at load time by a static initialiser and are read-only after.
#include "gf256.h"

#include <string.h>

#include <utility>
#include <vector>

#include "ec_mi355.h"

namespace ec {
namespace {

struct Tables {
  uint8_t exp[512];  // exp[i] = 2^i, doubled so that exp[log a + log b] needs no mod
  uint8_t log[256];  // log[0] unused
  Tables() {
    unsigned x = 1;
    for (int i = 0; i < 255; ++i) {
      exp[i] = (uint8_t)x;
      exp[i + 255] = (uint8_t)x;
      log[x] = (uint8_t)i;
      x <<= 1;
      if (x & 0x100u) x ^= 0x11Du;
    }
    exp[510] = exp[0];
    exp[511] = exp[1];
    log[0] = 0;
  }
};

const Tables& tables() {
  static const Tables t;
  return t;
}

}  // namespace

uint8_t gf_mul(uint8_t a, uint8_t b) {
  if (a == 0 || b == 0) return 0;
  const Tables& t = tables();
  return t.exp[t.log[a] + t.log[b]];
}

uint8_t gf_inv(uint8_t a) {
  if (a == 0) return 0;
  const Tables& t = tables();
  return t.exp[255 - t.log[a]];
}

PermTab perm_tab(uint8_t c) {
  uint8_t t0[8], t1[8], t2[4];
  for (int a = 0; a < 8; ++a) {
    t0[a] = gf_mul(c, (uint8_t)a);
    t1[a] = gf_mul(c, (uint8_t)(a << 3));
  }
  for (int a = 0; a < 4; ++a) t2[a] = gf_mul(c, (uint8_t)(a << 6));
  auto pack = [](const uint8_t* b) {
    return (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) |
           ((uint32_t)b[3] << 24);
  };
  PermTab p;
  p.lo0 = pack(t0);
  p.hi0 = pack(t0 + 4);
  p.lo1 = pack(t1);
  p.hi1 = pack(t1 + 4);
  p.t2 = pack(t2);
  return p;
}

int gf_invert(const uint8_t* in, uint8_t* out, int n) {
  std::vector<uint8_t> a(in, in + (size_t)n * n);
  memset(out, 0, (size_t)n * n);
  for (int i = 0; i < n; ++i) out[i * n + i] = 1;
  for (int c = 0; c < n; ++c) {
    int p = c;
    while (p < n && a[(size_t)p * n + c] == 0) ++p;
    if (p == n) return EC_ESINGULAR;
    if (p != c)
      for (int j = 0; j < n; ++j) {
        std::swap(a[(size_t)c * n + j], a[(size_t)p * n + j]);
        std::swap(out[(size_t)c * n + j], out[(size_t)p * n + j]);
      }
    const uint8_t s = gf_inv(a[(size_t)c * n + c]);
    for (int j = 0; j < n; ++j) {
      a[(size_t)c * n + j] = gf_mul(a[(size_t)c * n + j], s);
      out[(size_t)c * n + j] = gf_mul(out[(size_t)c * n + j], s);
    }
    for (int r = 0; r < n; ++r) {
      const uint8_t f = a[(size_t)r * n + c];
      if (r == c || f == 0) continue;
      for (int j = 0; j < n; ++j) {
        a[(size_t)r * n + j] ^= gf_mul(f, a[(size_t)c * n + j]);
        out[(size_t)r * n + j] ^= gf_mul(f, out[(size_t)c * n + j]);
      }
    }
  }
  return EC_OK;
}

}  // namespace ec

extern "C" {

int ec_abi_version(void) { return EC_ABI_VERSION; }

const char* ec_strerror(int status) {
  switch (status) {
    case EC_OK: return "success";
    case EC_EINVAL: return "invalid argument";
    case EC_EALIGN: return "pointer or size not 16-byte aligned";
    case EC_ESINGULAR: return "matrix singular or too many erasures";
    case EC_EHIP: return "HIP runtime error";
    case EC_ERANGE: return "k, m or length beyond supported limits";
    default: return "unknown status";
  }
}

uint8_t ec_gf_mul(uint8_t a, uint8_t b) { return ec::gf_mul(a, b); }

uint8_t ec_gf_inv(uint8_t a) { return ec::gf_inv(a); }

int ec_cauchy_matrix(int k, int m, uint8_t* out) {
  if (!out || k < 1 || m < 1) return EC_EINVAL;
  if (k + m > 256) return EC_ERANGE;
  for (int i = 0; i < m; ++i)
    for (int j = 0; j < k; ++j) out[i * k + j] = ec::gf_inv((uint8_t)((k + i) ^ j));
  return EC_OK;
}

int ec_gf_invert(const uint8_t* in, uint8_t* out, int n) {
  if (!in || !out || n < 1) return EC_EINVAL;
  if (n > 256) return EC_ERANGE;
  return ec::gf_invert(in, out, n);
}

int ec_decode_matrix(const uint8_t* coeff, int k, int m, const int* erased,
                     int n_erased, int* survivors, uint8_t* rows) {
  if (!coeff || !survivors || k < 1 || m < 0 || n_erased < 0) return EC_EINVAL;
  if (n_erased > 0 && (!erased || !rows)) return EC_EINVAL;
  if (k + m > 256) return EC_ERANGE;
  if (n_erased > m) return EC_ESINGULAR;
  const int n = k + m;
  std::vector<char> lost(n, 0);
  for (int e = 0; e < n_erased; ++e) {
    if (erased[e] < 0 || erased[e] >= n || lost[erased[e]]) return EC_EINVAL;
    lost[erased[e]] = 1;
  }
  int ns = 0;
  for (int g = 0; g < n && ns < k; ++g)
    if (!lost[g]) survivors[ns++] = g;
  // Generator row g: unit row for a data shard, Cauchy row for a parity shard.
  auto gen = [&](int g, uint8_t* row) {
    if (g < k) {
      memset(row, 0, (size_t)k);
      row[g] = 1;
    } else {
      memcpy(row, coeff + (size_t)(g - k) * k, (size_t)k);
    }
  };
  std::vector<uint8_t> gs((size_t)k * k), inv((size_t)k * k), row(k);
  for (int s = 0; s < k; ++s) gen(survivors[s], &gs[(size_t)s * k]);
  const int st = ec::gf_invert(gs.data(), inv.data(), k);
  if (st != EC_OK) return st;
  // lost_e = G[e] . data = (G[e] . inv(G_S)) . survivors
  for (int e = 0; e < n_erased; ++e) {
    gen(erased[e], row.data());
    for (int s = 0; s < k; ++s) {
      uint8_t acc = 0;
      for (int t = 0; t < k; ++t) acc ^= ec::gf_mul(row[t], inv[(size_t)t * k + s]);
      rows[(size_t)e * k + s] = acc;
    }
  }
  return EC_OK;
}

}  // extern "C"
