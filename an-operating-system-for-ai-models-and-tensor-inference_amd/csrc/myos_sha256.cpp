// SHA-256 of a file (FIPS 180-4), for the run fingerprint's model_sha256
// field (fingerprint.rs:63-206 keeps it; the reference leaves it null). The
// round constants and initial hash are the first 32 bits of the fractional
// parts of the cube roots of the first 64 primes and of the square roots of
// the first 8 (FIPS 180-4 sections 4.2.2 and 5.3.3), derived here once in
// long double rather than typed in.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/myos_hip.h"

namespace {

uint32_t K[64], H0[8];
std::once_flag g_once;

uint32_t frac32(long double v) {
  const long double f = v - floorl(v);
  return (uint32_t)floorl(f * 4294967296.0L);
}

void init_constants() {
  int n = 0;
  for (int p = 2; n < 64; p++) {
    bool prime = true;
    for (int d = 2; d * d <= p; d++)
      if (p % d == 0) {
        prime = false;
        break;
      }
    if (!prime) continue;
    if (n < 8) H0[n] = frac32(sqrtl((long double)p));
    K[n++] = frac32(cbrtl((long double)p));
  }
}

inline uint32_t rotr(uint32_t x, int r) { return (x >> r) | (x << (32 - r)); }

void compress(uint32_t h[8], const uint8_t *blk) {
  uint32_t w[64];
  for (int i = 0; i < 16; i++)
    w[i] = (uint32_t)blk[4 * i] << 24 | (uint32_t)blk[4 * i + 1] << 16 |
           (uint32_t)blk[4 * i + 2] << 8 | blk[4 * i + 3];
  for (int i = 16; i < 64; i++) {
    const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
    const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
    w[i] = w[i - 16] + s0 + w[i - 7] + s1;
  }
  uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], k = h[7];
  for (int i = 0; i < 64; i++) {
    const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
    const uint32_t ch = (e & f) ^ (~e & g);
    const uint32_t t1 = k + S1 + ch + K[i] + w[i];
    const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
    const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
    const uint32_t t2 = S0 + maj;
    k = g;
    g = f;
    f = e;
    e = d + t1;
    d = c;
    c = b;
    b = a;
    a = t1 + t2;
  }
  h[0] += a;
  h[1] += b;
  h[2] += c;
  h[3] += d;
  h[4] += e;
  h[5] += f;
  h[6] += g;
  h[7] += k;
}

}  // namespace

extern "C" int myos_sha256_file(const char *path, char *out_hex) {
  if (!path || !out_hex) return MYOS_E_ARG;
  std::call_once(g_once, init_constants);
  FILE *f = fopen(path, "rb");
  if (!f) return MYOS_E_IO;
  uint32_t h[8];
  memcpy(h, H0, sizeof h);
  static constexpr size_t kBuf = 1 << 20;
  uint8_t *buf = new uint8_t[kBuf + 128];
  uint64_t total = 0;
  size_t got;
  int rc = MYOS_OK;
  while ((got = fread(buf, 1, kBuf, f)) == kBuf) {
    for (size_t o = 0; o < kBuf; o += 64) compress(h, buf + o);
    total += kBuf;
  }
  if (ferror(f)) rc = MYOS_E_IO;
  fclose(f);
  if (rc == MYOS_OK) {
    // the tail, then 0x80, zeros and the bit length (big-endian) to a whole block
    total += got;
    size_t n = got;
    buf[n++] = 0x80;
    while (n % 64 != 56) buf[n++] = 0;
    const uint64_t bits = total * 8;
    for (int i = 7; i >= 0; i--) buf[n++] = (uint8_t)(bits >> (8 * i));
    for (size_t o = 0; o < n; o += 64) compress(h, buf + o);
    for (int i = 0; i < 8; i++) snprintf(out_hex + 8 * i, 9, "%08x", h[i]);
  }
  delete[] buf;
  return rc;
}
