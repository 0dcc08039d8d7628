// Seeded random-init writer for Qwen2.5-shaped BF16 SafeTensors files (the
// benchmark models: real checkpoints are not available offline).
//
// Element i of tensor `name` (i counted in row-major order):
//   key   = seed ^ FNV-1a64(name)
//   u(n)  = (splitmix64(key + (n + 1) * 0x9E3779B97F4A7C15) >> 11) * 2^-53
//   pair j = i / 2: r = sqrt(-2 ln(1 - u(2j))), a = 2 pi u(2j + 1)
//   z = r cos a (even i) or r sin a (odd i), in double
//   value = bf16_rne((float)(std * z))
// Norm gains ("*norm.weight") are 1.0. The stream is counter-based, so any
// split of the elements over threads writes the same bytes.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <thread>
#include <vector>

#include "../../include/myos_hip.h"

namespace {

uint64_t fnv1a64(const std::string &s) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 0x100000001b3ull;
  }
  return h;
}

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

inline double unit(uint64_t key, uint64_t n) {
  return (double)(mix64(key + (n + 1) * 0x9e3779b97f4a7c15ull) >> 11) * 0x1.0p-53;
}

inline uint16_t bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// elements [i0, i1) into out[0, i1 - i0); each Box-Muller pair's radius and
// angle are evaluated once for both of its elements
void fill_normal(uint16_t *out, size_t i0, size_t i1, uint64_t key, float std_dev) {
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = i0; i < i1;) {
    const uint64_t j = i / 2;
    const double r = sqrt(-2.0 * log(1.0 - unit(key, 2 * j)));
    const double a = two_pi * unit(key, 2 * j + 1);
    if (!(i & 1)) {
      out[i - i0] = bf16_rne((float)((double)std_dev * (r * cos(a))));
      if (++i == i1) break;
    }
    out[i - i0] = bf16_rne((float)((double)std_dev * (r * sin(a))));
    i++;
  }
}

struct T {
  std::string name;
  std::vector<size_t> shape;
  size_t numel() const {
    size_t n = 1;
    for (size_t d : shape) n *= d;
    return n;
  }
};

}  // namespace

extern "C" int myos_write_random_qwen25(const char *path, const myos_block_shape *s,
                                        uint64_t seed, float std_dev, int threads) {
  if (!path || !s) return MYOS_E_ARG;
  if (!s->hidden || !s->num_q_heads || !s->num_kv_heads || !s->head_dim || !s->intermediate ||
      !s->vocab || !s->num_layers)
    return MYOS_E_SHAPE;
  const size_t H = s->hidden, I = s->intermediate, V = s->vocab;
  const size_t Q = s->num_q_heads * s->head_dim, KD = s->num_kv_heads * s->head_dim;
  std::vector<T> ts;
  ts.push_back({"model.embed_tokens.weight", {V, H}});
  ts.push_back({"model.norm.weight", {H}});
  if (!s->tied_head) ts.push_back({"lm_head.weight", {V, H}});
  const char *suf[12] = {"input_layernorm.weight", "self_attn.q_proj.weight",
                         "self_attn.q_proj.bias",  "self_attn.k_proj.weight",
                         "self_attn.k_proj.bias",  "self_attn.v_proj.weight",
                         "self_attn.v_proj.bias",  "self_attn.o_proj.weight",
                         "post_attention_layernorm.weight", "mlp.gate_proj.weight",
                         "mlp.up_proj.weight",     "mlp.down_proj.weight"};
  const std::vector<size_t> shp[12] = {{H}, {Q, H}, {Q}, {KD, H}, {KD}, {KD, H},
                                       {KD}, {H, Q}, {H}, {I, H}, {I, H}, {H, I}};
  for (size_t l = 0; l < s->num_layers; l++)
    for (int j = 0; j < 12; j++)
      ts.push_back({"model.layers." + std::to_string(l) + "." + suf[j], shp[j]});

  std::string hdr = "{";
  size_t off = 0;
  for (size_t i = 0; i < ts.size(); i++) {
    const size_t nb = ts[i].numel() * 2;
    hdr += (i ? "," : "") + std::string("\"") + ts[i].name + "\":{\"dtype\":\"BF16\",\"shape\":[";
    for (size_t d = 0; d < ts[i].shape.size(); d++)
      hdr += (d ? "," : "") + std::to_string(ts[i].shape[d]);
    hdr += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + nb) + "]}";
    off += nb;
  }
  hdr += "}";
  while (hdr.size() % 8) hdr += ' ';
  FILE *f = fopen(path, "wb");
  if (!f) return MYOS_E_IO;
  uint64_t n = hdr.size();
  uint8_t le[8];
  for (int i = 0; i < 8; i++) le[i] = (uint8_t)(n >> (8 * i));
  bool ok = fwrite(le, 1, 8, f) == 8 && fwrite(hdr.data(), 1, hdr.size(), f) == hdr.size();
  const int nt = threads < 1 ? 1 : (threads > 256 ? 256 : threads);
  const size_t chunk = 1ull << 24;  // elements per write
  std::vector<uint16_t> buf(chunk);
  for (size_t t = 0; t < ts.size() && ok; t++) {
    const size_t total = ts[t].numel();
    const bool gain = ts[t].name.size() >= 11 &&
                      ts[t].name.compare(ts[t].name.size() - 11, 11, "norm.weight") == 0;
    const uint64_t key = seed ^ fnv1a64(ts[t].name);
    for (size_t c0 = 0; c0 < total && ok; c0 += chunk) {
      const size_t c1 = c0 + chunk < total ? c0 + chunk : total;
      if (gain) {
        for (size_t i = c0; i < c1; i++) buf[i - c0] = 0x3F80;  // 1.0
      } else {
        std::vector<std::thread> pool;
        const size_t per = (c1 - c0 + nt - 1) / nt;
        for (int w = 0; w < nt; w++) {
          const size_t a = c0 + w * per, b = a + per < c1 ? a + per : c1;
          if (a >= b) break;
          pool.emplace_back([&, a, b] { fill_normal(buf.data() + (a - c0), a, b, key, std_dev); });
        }
        for (auto &th : pool) th.join();
      }
      ok = fwrite(buf.data(), 2, c1 - c0, f) == c1 - c0;
    }
  }
  if (fclose(f) != 0) ok = false;
  return ok ? MYOS_OK : MYOS_E_IO;
}
