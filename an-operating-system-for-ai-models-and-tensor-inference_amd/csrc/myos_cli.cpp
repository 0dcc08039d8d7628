// `myos`: the runtime CLI of the reference (crates/runtime/src/main.rs) over
// the MI355X library. Same flags, stdout lines and output files:
//
//   --weights PATH (or MYOS_WEIGHTS)  SafeTensors file, qwen25_layout keys
//   --block-fixture                   the in-process miniature block
//                                     (qwen25_block.rs:788-840)
//   --steps N                         greedy steps (default 4, main.rs:353-357)
//   --threads N                       recorded (1..64, default 8); the device
//                                     path has no host GEMV workers
//   --prompt-ids PATH                 whitespace-separated u32 prompt (default [0])
//   --ref-ids PATH                    prints CORRECT: PASS / FAIL first_diff@i
//   --fingerprint-dir DIR             run_fingerprint.json, token_ids.txt and
//                                     metrics.json go here (default runs/<id>)
//
//   --arena-s1 [--warmup W] [--repeats R]
//                                     the W/R showdown harness (arena.rs): W + R
//                                     fresh child processes, medians, DET and
//                                     CORRECT gates (myos_arena.cpp); --steps
//                                     defaults to 128 there
//
// and, for the device: --model-shape 1.5b|7b, --kv f32|bf16,
// --decode-path auto|kernels|persistent|streamed, --no-graph, and two verification
// passes run after the timed decode (outside its timing): --gaps re-runs the
// decode step by step and records every step's top-1 / top-2 logit gap;
// --teacher-forced (with --ref-ids) feeds the reference ids instead and
// reports how many steps' greedy ids agree with them. --no-hash leaves
// model_sha256 null (the arena's children: the parent hashes once). The arena's llama.cpp
// cost card (--cost-card) compares against a CPU competitor and is refused.
//
// run_fingerprint.json keeps the reference's fields (fingerprint.rs:161-203)
// with device = the GPU and model_sha256 = the weights file's SHA-256;
// metrics.json keeps meter.rs:183-232's fields, with t_prefill / t_decode
// around the same boundaries (main.rs:515-545) and M_peak from a 20 ms VmRSS
// sampler (meter.rs:679-723), plus device fields: arch, HBM peak, algorithmic
// bytes per decode token, achieved GB/s and the HBM roofline fraction.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <errno.h>
#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <cmath>
#include <fstream>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

#include "../../include/myos_hip.h"
#include "myos_arena.h"

namespace {

const char *kUsage =
    "myos [--weights PATH] [--block-fixture] [--steps N] [--threads N] [--fingerprint-dir DIR] "
    "[--prompt-ids PATH] [--ref-ids PATH] [--arena-s1] [--warmup N] [--repeats N] "
    "[--model-shape 1.5b|7b] [--kv f32|bf16] [--decode-path auto|kernels|persistent|streamed] "
    "[--no-graph] [--gaps] [--teacher-forced] [--no-hash]";

constexpr double kHbmPeakGBps = 8000.0;  // MI355X HBM3E

struct Cli {
  std::string weights, fingerprint_dir, prompt_ids, ref_ids;
  bool has_weights = false, has_fp = false, has_prompt = false, has_ref = false;
  bool block_fixture = false;
  size_t steps = 4;
  bool has_steps = false;
  size_t threads = 8;
  bool has_threads = false;
  int shape = MYOS_SHAPE_QWEN25_1_5B;
  int kv = MYOS_KV_F32;
  int decode = MYOS_DECODE_AUTO;
  bool has_shape = false, has_kv = false, has_decode = false;
  bool arena = false, has_warmup = false, has_repeats = false;
  size_t warmup = 3, repeats = 5;
  bool no_graph = false, gaps = false, teacher = false, no_hash = false;
};

const char *flag_noun(const std::string &name) {
  if (name == "--steps" || name == "--threads" || name == "--repeats") return "a positive integer";
  if (name == "--warmup") return "a non-negative integer";
  if (name == "--model-shape") return "1.5b or 7b";
  if (name == "--kv") return "f32 or bf16";
  if (name == "--decode-path") return "auto, kernels, persistent or streamed";
  return "a path";
}

// `--name VALUE` or `--name=VALUE` (main.rs:373-397); 1 matched, 0 not this
// flag, -1 error (message in err)
int match_flag(const std::string &arg, const std::string &name, int &i, int argc, char **argv,
               std::string &out, std::string &err) {
  const std::string prefix = name + "=";
  if (arg.compare(0, prefix.size(), prefix) == 0) {
    out = arg.substr(prefix.size());
    if (out.empty()) {
      err = name + " needs " + flag_noun(name);
      return -1;
    }
    return 1;
  }
  if (arg == name) {
    if (i + 1 >= argc || argv[i + 1][0] == '\0') {
      err = name + " needs " + flag_noun(name);
      return -1;
    }
    out = argv[++i];
    return 1;
  }
  return 0;
}

bool parse_positive(const std::string &v, size_t &out) {
  if (v.empty()) return false;
  char *end = nullptr;
  const unsigned long long n = strtoull(v.c_str(), &end, 10);
  if (*end != '\0' || v[0] == '-' || n == 0) return false;
  out = (size_t)n;
  return true;
}

// parse_cli, main.rs:237-371 (arena flags refused)
int parse_cli(int argc, char **argv, Cli &c, std::string &err) {
  for (int i = 1; i < argc; i++) {
    const std::string arg = argv[i];
    std::string v;
    int r;
    if (arg == "--block-fixture") {
      if (c.block_fixture) return err = "--block-fixture was given more than once", -1;
      c.block_fixture = true;
      continue;
    }
    bool *sw = arg == "--arena-s1" ? &c.arena : arg == "--no-graph" ? &c.no_graph
             : arg == "--gaps" ? &c.gaps : arg == "--teacher-forced" ? &c.teacher
             : arg == "--no-hash" ? &c.no_hash : nullptr;
    if (sw) {
      if (*sw) return err = arg + " was given more than once", -1;
      *sw = true;
      continue;
    }
    if (arg.rfind("--cost-card", 0) == 0)
      return err = arg + ": the llama.cpp cost card is not part of the device build", -1;
    if ((r = match_flag(arg, "--warmup", i, argc, argv, v, err)) != 0) {
      if (r < 0) return -1;
      if (c.has_warmup) return err = "--warmup was given more than once", -1;
      char *end = nullptr;
      const unsigned long long n = strtoull(v.c_str(), &end, 10);
      if (v.empty() || *end != '\0' || v[0] == '-')
        return err = "--warmup needs a non-negative integer, got `" + v + "`", -1;
      c.warmup = (size_t)n;
      c.has_warmup = true;
      continue;
    }
    if ((r = match_flag(arg, "--repeats", i, argc, argv, v, err)) != 0) {
      if (r < 0) return -1;
      if (c.has_repeats) return err = "--repeats was given more than once", -1;
      if (!parse_positive(v, c.repeats))
        return err = "--repeats needs a positive integer, got `" + v + "`", -1;
      c.has_repeats = true;
      continue;
    }
    struct {
      const char *name;
      std::string *dst;
      bool *seen;
    } paths[] = {{"--weights", &c.weights, &c.has_weights},
                 {"--fingerprint-dir", &c.fingerprint_dir, &c.has_fp},
                 {"--prompt-ids", &c.prompt_ids, &c.has_prompt},
                 {"--ref-ids", &c.ref_ids, &c.has_ref}};
    bool done = false;
    for (auto &p : paths) {
      r = match_flag(arg, p.name, i, argc, argv, v, err);
      if (r < 0) return -1;
      if (r == 1) {
        if (*p.seen) return err = std::string(p.name) + " was given more than once", -1;
        *p.dst = v;
        *p.seen = true;
        done = true;
        break;
      }
    }
    if (done) continue;
    if ((r = match_flag(arg, "--steps", i, argc, argv, v, err)) != 0) {
      if (r < 0) return -1;
      if (c.has_steps) return err = "--steps was given more than once", -1;
      if (!parse_positive(v, c.steps))
        return err = "--steps needs a positive integer, got `" + v + "`", -1;
      c.has_steps = true;
      continue;
    }
    if ((r = match_flag(arg, "--threads", i, argc, argv, v, err)) != 0) {
      if (r < 0) return -1;
      if (c.has_threads) return err = "--threads was given more than once", -1;
      if (!parse_positive(v, c.threads) || c.threads > 64)
        return err = "--threads needs an integer from 1 to 64, got `" + v + "`", -1;
      c.has_threads = true;
      continue;
    }
    if ((r = match_flag(arg, "--model-shape", i, argc, argv, v, err)) != 0) {
      if (r < 0) return -1;
      if (v == "1.5b") c.shape = MYOS_SHAPE_QWEN25_1_5B;
      else if (v == "7b") c.shape = MYOS_SHAPE_QWEN25_7B;
      else return err = "--model-shape needs 1.5b or 7b, got `" + v + "`", -1;
      c.has_shape = true;
      continue;
    }
    if ((r = match_flag(arg, "--kv", i, argc, argv, v, err)) != 0) {
      if (r < 0) return -1;
      if (v == "f32") c.kv = MYOS_KV_F32;
      else if (v == "bf16") c.kv = MYOS_KV_BF16;
      else return err = "--kv needs f32 or bf16, got `" + v + "`", -1;
      c.has_kv = true;
      continue;
    }
    if ((r = match_flag(arg, "--decode-path", i, argc, argv, v, err)) != 0) {
      if (r < 0) return -1;
      if (v == "auto") c.decode = MYOS_DECODE_AUTO;
      else if (v == "kernels") c.decode = MYOS_DECODE_KERNELS;
      else if (v == "persistent") c.decode = MYOS_DECODE_PERSISTENT;
      else if (v == "streamed") c.decode = MYOS_DECODE_STREAMED;
      else return err = "--decode-path needs auto, kernels, persistent or streamed, got `" + v + "`", -1;
      c.has_decode = true;
      continue;
    }
    return err = "unknown argument `" + arg + "`", -1;
  }
  if (!c.has_weights) {
    const char *env = getenv("MYOS_WEIGHTS");  // selected_weights_path, main.rs:439-446
    if (env && env[0]) {
      c.weights = env;
      c.has_weights = true;
    }
  }
  if (c.has_fp && !c.has_weights && !c.block_fixture)
    return err = "--fingerprint-dir needs --weights or --block-fixture", -1;
  if (c.has_prompt && !c.has_weights) return err = "--prompt-ids needs --weights", -1;
  if (c.has_prompt && c.block_fixture)
    return err = "--prompt-ids cannot be combined with --block-fixture", -1;
  // main.rs:339-352
  if (c.arena) {
    if (c.block_fixture) return err = "--arena-s1 cannot be combined with --block-fixture", -1;
    if (!c.has_weights) return err = "--arena-s1 needs --weights", -1;
    if (!c.has_prompt) return err = "--arena-s1 needs --prompt-ids", -1;
    if (!c.has_ref) return err = "--arena-s1 needs --ref-ids", -1;
    if (!c.has_steps) c.steps = 128;
  } else if (c.has_warmup || c.has_repeats) {
    return err = "--warmup and --repeats need --arena-s1", -1;
  }
  if (c.teacher && !c.has_ref) return err = "--teacher-forced needs --ref-ids", -1;
  return 0;
}

// read_token_ids / parse_token_ids, main.rs:645-669
int read_token_ids(const std::string &path, std::vector<uint32_t> &ids, std::string &err) {
  std::ifstream f(path);
  if (!f) return err = path + ": cannot read", -1;
  std::string tok;
  while (f >> tok) {
    char *end = nullptr;
    const unsigned long long v = strtoull(tok.c_str(), &end, 10);
    if (*end != '\0' || tok[0] == '-' || v > 0xffffffffull)
      return err = path + ": `" + tok + "` is not a u32", -1;
    ids.push_back((uint32_t)v);
  }
  if (ids.empty()) return err = path + ": file is empty", -1;
  return 0;
}

// correct_line, main.rs:672-686
std::string correct_line(const std::vector<uint32_t> &got, const std::vector<uint32_t> &ref) {
  if (got.size() != ref.size())
    return "CORRECT: FAIL length mismatch got=" + std::to_string(got.size()) +
           " ref=" + std::to_string(ref.size());
  for (size_t i = 0; i < got.size(); i++)
    if (got[i] != ref[i])
      return "CORRECT: FAIL first_diff@" + std::to_string(i) + ": got=" + std::to_string(got[i]) +
             " ref=" + std::to_string(ref[i]);
  return "CORRECT: PASS";
}

std::string ids_list(const std::vector<uint32_t> &ids) {
  std::string s = "[";
  for (size_t i = 0; i < ids.size(); i++) s += (i ? ", " : "") + std::to_string(ids[i]);
  return s + "]";
}

std::string json_str(const std::string &v) {
  std::string o = "\"";
  for (char ch : v) {
    if (ch == '"' || ch == '\\') o += '\\', o += ch;
    else if (ch == '\n') o += "\\n";
    else if ((unsigned char)ch < 0x20) {
      char b[8];
      snprintf(b, sizeof b, "\\u%04x", ch);
      o += b;
    } else o += ch;
  }
  return o + "\"";
}
std::string json_num(double v) {
  char b[64];
  snprintf(b, sizeof b, "%.9g", v);
  return b;
}

int mkdirs(const std::string &dir) {
  std::string cur;
  std::stringstream ss(dir);
  std::string part;
  if (!dir.empty() && dir[0] == '/') cur = "/";
  while (std::getline(ss, part, '/')) {
    if (part.empty()) continue;
    cur += part + "/";
    if (mkdir(cur.c_str(), 0755) != 0 && errno != EEXIST) return -1;
  }
  return 0;
}

// VmRSS / VmHWM from /proc/self/status, KiB (meter.rs vm_rss_kib)
long proc_kib(const char *key) {
  std::ifstream f("/proc/self/status");
  std::string line;
  const size_t n = strlen(key);
  while (std::getline(f, line))
    if (line.compare(0, n, key) == 0) return atol(line.c_str() + n);
  return -1;
}

std::string device_name() {
  hipDeviceProp_t p;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess)
    return "hip";
  return std::string(p.name) + " (" + p.gcnArchName + ")";
}

// The reference's miniature block (qwen25_block.rs:788-840): hidden 2,
// vocab 4, one layer, eps 0; token 0 -> logits [1, 2, 0, -1], greedy [1, 1, 1, 1].
// Written as a BF16 SafeTensors file so it goes through the same loader.
int write_block_fixture(const std::string &path) {
  struct T {
    std::string name;
    std::vector<size_t> shape;
    std::vector<float> v;
  };
  auto z = [](size_t n) { return std::vector<float>(n, 0.f); };
  std::vector<T> ts = {
      {"model.embed_tokens.weight", {4, 2}, {1, 1, 2, 0, 0, 4, -1, 0}},
      {"model.norm.weight", {2}, {1, 0}},
      {"model.layers.0.input_layernorm.weight", {2}, {1, 1}},
      {"model.layers.0.self_attn.q_proj.weight", {4, 2}, z(8)},
      {"model.layers.0.self_attn.q_proj.bias", {4}, {0.5f, 0, 0, 0.25f}},
      {"model.layers.0.self_attn.k_proj.weight", {2, 2}, z(4)},
      {"model.layers.0.self_attn.k_proj.bias", {2}, z(2)},
      {"model.layers.0.self_attn.v_proj.weight", {2, 2}, z(4)},
      {"model.layers.0.self_attn.v_proj.bias", {2}, {1, 0}},
      {"model.layers.0.self_attn.o_proj.weight", {2, 4}, {1, 0, 0, 0, 1, 0, 0, 0}},
      {"model.layers.0.post_attention_layernorm.weight", {2}, {1, 1}},
      {"model.layers.0.mlp.gate_proj.weight", {2, 2}, z(4)},
      {"model.layers.0.mlp.up_proj.weight", {2, 2}, z(4)},
      {"model.layers.0.mlp.down_proj.weight", {2, 2}, z(4)},
  };
  std::string hdr = "{";
  size_t off = 0;
  for (size_t i = 0; i < ts.size(); i++) {
    const size_t nb = ts[i].v.size() * 2;
    std::string shp;
    for (size_t k = 0; k < ts[i].shape.size(); k++) shp += (k ? "," : "") + std::to_string(ts[i].shape[k]);
    hdr += (i ? "," : "") + json_str(ts[i].name) + ":{\"dtype\":\"BF16\",\"shape\":[" + shp +
           "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + nb) + "]}";
    off += nb;
  }
  hdr += "}";
  while (hdr.size() % 8) hdr += ' ';
  FILE *f = fopen(path.c_str(), "wb");
  if (!f) return -1;
  const uint64_t hl = hdr.size();
  fwrite(&hl, 8, 1, f);
  fwrite(hdr.data(), 1, hdr.size(), f);
  for (auto &t : ts)
    for (float x : t.v) {
      uint32_t u;
      memcpy(&u, &x, 4);
      const uint16_t b = (uint16_t)(u >> 16);  // every fixture value is exact in bf16
      fwrite(&b, 2, 1, f);
    }
  return fclose(f) == 0 ? 0 : -1;
}

std::string cmdline(int argc, char **argv) {
  std::string s;
  for (int i = 0; i < argc; i++) s += (i ? " " : "") + std::string(argv[i]);
  return s;
}

struct Run {
  std::vector<uint32_t> prompt, tokens;
  double t_load_s = 0, t_prefill_s = 0, t_decode_s = 0;
  double dev_prefill_ms = 0, dev_decode_ms = 0;
  long rss_after_load = -1, peak = -1, hwm = -1;
  int decode_path = MYOS_DECODE_KERNELS;
  size_t weight_bytes = 0, kv_bytes = 0;
  bool graph = true;
  std::string sha256;  // empty: not hashed (block fixture) or unreadable
  // verification pass (--gaps / --teacher-forced), outside the timed region
  std::string verify_mode;
  std::vector<uint32_t> verify_ids;  // greedy id of each step's input logits
  std::vector<double> gaps;          // their top-1 / top-2 gap
};

// RssSampler, meter.rs:679-723: VmRSS polled every 20 ms on a thread; the
// peak is the largest sample (taken from after load to after decode)
struct RssSampler {
  std::atomic<bool> stop{false};
  std::atomic<long> peak{-1};
  std::thread th;
  void start() {
    peak = proc_kib("VmRSS:");
    th = std::thread([this] {
      while (!stop.load()) {
        const long v = proc_kib("VmRSS:");
        if (v > peak.load()) peak = v;
        std::this_thread::sleep_for(std::chrono::milliseconds(20));
      }
    });
  }
  long finish() {
    stop = true;
    if (th.joinable()) th.join();
    const long v = proc_kib("VmRSS:");
    return v > peak.load() ? v : peak.load();
  }
};

// greedy id and top-1 / top-2 gap of the logits the last forward left
int logits_top2(myos_model *m, size_t vocab, std::vector<float> &buf, uint32_t *id, double *gap) {
  buf.resize(vocab);
  int rc = myos_copy_logits(m, buf.data(), vocab);
  if (rc) return rc;
  // greedy_token (model_core/src/lib.rs:157-167): strict >, lowest index on ties
  float best = -INFINITY;
  uint32_t bi = 0;
  for (size_t i = 0; i < vocab; i++)
    if (buf[i] > best) best = buf[i], bi = (uint32_t)i;
  float second = -INFINITY;
  for (size_t i = 0; i < vocab; i++)
    if (i != bi && buf[i] > second) second = buf[i];
  *id = bi;
  *gap = (double)best - (double)second;
  return MYOS_OK;
}

// decode_bf16_timed (main.rs:515-545): open (t_load), then prefill (t_prefill,
// ending before the first new token), then greedy_decode (t_decode); then,
// untimed, the verification pass when asked for
int decode_timed(const std::string &path, const myos_block_shape &shape, const Cli &c,
                 const std::vector<uint32_t> *teacher, Run &r) {
  using clk = std::chrono::steady_clock;
  const size_t max_seq = r.prompt.size() + r.tokens.size();
  myos_model *m = nullptr;
  auto t0 = clk::now();
  int rc = myos_model_open(path.c_str(), &shape, c.kv, max_seq, &m);
  if (rc) return rc;
  r.t_load_s = std::chrono::duration<double>(clk::now() - t0).count();
  r.rss_after_load = proc_kib("VmRSS:");
  if (c.decode != MYOS_DECODE_AUTO && (rc = myos_set_decode_mode(m, c.decode)) != MYOS_OK) {
    myos_model_close(m);
    return rc;
  }
  if (c.no_graph && (rc = myos_set_graph(m, 0)) != MYOS_OK) {
    myos_model_close(m);
    return rc;
  }
  r.graph = !c.no_graph;
  r.decode_path = myos_decode_path(m);
  RssSampler rss;
  rss.start();
  auto t1 = clk::now();
  rc = myos_prefill(m, r.prompt.data(), r.prompt.size());
  if (!rc) rc = myos_stream_sync(nullptr);
  auto t2 = clk::now();
  if (!rc) rc = myos_greedy_decode(m, r.tokens.size(), r.tokens.data());
  auto t3 = clk::now();
  r.peak = rss.finish();
  r.t_prefill_s = std::chrono::duration<double>(t2 - t1).count();
  r.t_decode_s = std::chrono::duration<double>(t3 - t2).count();
  r.dev_prefill_ms = myos_last_prefill_ms(m);
  r.dev_decode_ms = myos_last_decode_ms(m);
  r.weight_bytes = myos_weight_bytes(m);
  r.kv_bytes = myos_kv_bytes(m);
  if (!rc && (c.gaps || c.teacher)) {
    // the same decode again, one step per call, reading each step's logits:
    // fed the reference ids (--teacher-forced) or its own greedy ids
    r.verify_mode = c.teacher ? "teacher-forced" : "greedy";
    rc = myos_cache_clear(m);
    if (!rc) rc = myos_prefill(m, r.prompt.data(), r.prompt.size());
    std::vector<float> buf;
    for (size_t i = 0; !rc && i < r.tokens.size(); i++) {
      uint32_t id;
      double gap;
      rc = logits_top2(m, shape.vocab, buf, &id, &gap);
      if (rc) break;
      r.verify_ids.push_back(id);
      r.gaps.push_back(gap);
      uint32_t out;
      if (c.teacher) {
        const uint32_t feed = i < teacher->size() ? (*teacher)[i] : id;
        rc = myos_decode_forced(m, &feed, 1, &out);
      } else {
        rc = myos_greedy_decode(m, 1, &out);
      }
    }
  }
  r.hwm = proc_kib("VmHWM:");
  myos_model_close(m);
  return rc;
}

// algorithmic HBM bytes of one decode token at sequence length seq: every
// bf16 weight the step streams (all layers, final norm, the head, one embed
// row) plus the K/V rows attention reads
double decode_token_bytes(const myos_block_shape &s, double seq, int kv) {
  const double H = (double)s.hidden, I = (double)s.intermediate, V = (double)s.vocab;
  const double Q = (double)(s.num_q_heads * s.head_dim), KD = (double)(s.num_kv_heads * s.head_dim);
  const double per_layer = 2 * H + Q * H + Q + 2 * (KD * H + KD) + H * Q + 3 * I * H;
  const double w = 2 * ((double)s.num_layers * per_layer + H + V * H + H);
  const double kvb = (double)s.num_layers * 2 * KD * seq * (kv == MYOS_KV_BF16 ? 2 : 4);
  return w + kvb;
}

int write_text(const std::string &dir, const char *name, const std::string &text) {
  if (mkdirs(dir)) return -1;
  std::ofstream f(dir + "/" + name);
  f << text;
  return f ? 0 : -1;
}

// the name run_fingerprint.json and metrics.json give a decode path
const char *decode_path_name(int dp) {
  return dp == MYOS_DECODE_PERSISTENT ? "persistent" : dp == MYOS_DECODE_STREAMED ? "streamed" : "kernels";
}

// run_fingerprint.json (fingerprint.rs:161-203) + device fields
std::string fingerprint_json(const Cli &c, const myos_block_shape &s, bool weights, bool pinned,
                             const Run &r, int argc, char **argv) {
  const char *layout = !weights ? "block-fixture" : pinned ? "qwen25_1_5b" : "not-qwen25-1.5b";
  const std::string model_id = weights && pinned ? json_str("Qwen/Qwen2.5-1.5B-Instruct") : "null";
  const char *dp = decode_path_name(r.decode_path);
  std::vector<std::pair<std::string, std::string>> f = {
      {"model_id", model_id},
      {"model_sha256", r.sha256.empty() ? "null" : json_str(r.sha256)},
      {"fmt", json_str(weights ? "safetensors" : "in-process")},
      {"quant_or_dtype", json_str("bf16")},
      {"acc_path", json_str("bf16_w_fp32_acc")},
      {"n_ctx", std::to_string(r.prompt.size() + r.tokens.size())},
      {"n_prompt", std::to_string(r.prompt.size())},
      {"n_gen", std::to_string(r.tokens.size())},
      {"batch", "1"},
      {"threads", std::to_string(c.threads)},
      {"gemv_pack", "false"},
      {"device", json_str(device_name())},
      {"deterministic", "true"},
      {"seed", "null"},
      {"commit", "null"},
      {"cmdline", json_str(cmdline(argc, argv))},
      {"scenario_id", json_str("S1")},
      {"run_id", json_str(weights ? "s1-weights" : "s1-block-fixture")},
      {"layout", json_str(layout)},
      {"num_layers", std::to_string(s.num_layers)},
      {"hidden_size", std::to_string(s.hidden)},
      {"intermediate_size", std::to_string(s.intermediate)},
      {"vocab_size", std::to_string(s.vocab)},
      {"prompt_token", std::to_string(r.prompt.empty() ? 0 : r.prompt[0])},
      {"decode_path", json_str(dp)},
      {"kv_dtype", json_str(c.kv == MYOS_KV_BF16 ? "bf16" : "f32")},
      {"build", json_str(myos_build_info())},
      {"graph", r.graph ? "true" : "false"},
      {"notes", json_str("Device run: weights uploaded once to HBM, prefill on MFMA (bf16 hi/lo "
                         "activation split), greedy decode on the GPU. threads is the recorded "
                         "--threads value; the device path has no host GEMV workers. "
                         "model_sha256 is the SHA-256 of the weights file.")},
  };
  std::string o = "{\n";
  for (size_t i = 0; i < f.size(); i++)
    o += "  \"" + f[i].first + "\": " + f[i].second + (i + 1 < f.size() ? ",\n" : "\n");
  return o + "}\n";
}

std::string arch_name() {
  hipDeviceProp_t p;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess)
    return "unknown";
  std::string a = p.gcnArchName;
  return a.substr(0, a.find(':'));
}

// metrics.json (meter.rs:183-232 + derive :48-78) + device fields
std::string metrics_json(const Cli &c, const myos_block_shape &shape, const Run &r, int correct,
                         const std::vector<uint32_t> *ref) {
  const double n_gen = (double)r.tokens.size(), n_prompt = (double)r.prompt.size();
  // bytes per decode token averaged over the steps (sequence n_prompt + 1 ..
  // n_prompt + n_gen), and what the device moved at its decode rate
  const double b_tok = decode_token_bytes(shape, n_prompt + (n_gen + 1) / 2, c.kv);
  const double dev_tok_s = r.dev_decode_ms > 0 ? n_gen / (r.dev_decode_ms * 1e-3) : 0;
  const double gbps = b_tok * dev_tok_s / 1e9;
  std::string gaps = "[", vids = "[";
  double min_gap = INFINITY;
  size_t agree = 0;
  long first_diff = -1;
  const std::vector<uint32_t> &want = r.verify_mode == "teacher-forced" && ref ? *ref : r.tokens;
  for (size_t i = 0; i < r.gaps.size(); i++) {
    gaps += (i ? ", " : "") + json_num(r.gaps[i]);
    vids += (i ? ", " : "") + std::to_string(r.verify_ids[i]);
    min_gap = std::min(min_gap, r.gaps[i]);
    if (i < want.size() && r.verify_ids[i] == want[i]) agree++;
    else if (first_diff < 0) first_diff = (long)i;
  }
  gaps += "]";
  vids += "]";
  const bool verified = !r.verify_mode.empty();
  auto mib = [](long k) { return k < 0 ? std::string("null") : json_num(k / 1024.0); };
  auto kib = [](long k) { return k < 0 ? std::string("null") : std::to_string(k); };
  std::vector<std::pair<std::string, std::string>> f = {
      {"scenario_id", json_str("S1")},
      {"threads", std::to_string(c.threads)},
      {"batch", "1"},
      {"quant_or_dtype", json_str("bf16")},
      {"acc_path", json_str("bf16_w_fp32_acc")},
      {"gemv_pack", "false"},
      {"n_prompt", std::to_string(r.prompt.size())},
      {"n_gen", std::to_string(r.tokens.size())},
      {"t_load_s", json_num(r.t_load_s)},
      {"t_prefill_s", json_num(r.t_prefill_s)},
      {"t_decode_s", json_num(r.t_decode_s)},
      {"T_decode_tok_s", r.t_decode_s > 0 ? json_num(n_gen / r.t_decode_s) : "null"},
      {"L_TTFT_ms", json_num(r.t_prefill_s * 1e3)},
      {"L_prefill_ms", json_num(r.t_prefill_s * 1e3)},
      {"L_TPOT_ms", n_gen > 0 ? json_num(r.t_decode_s * 1e3 / n_gen) : "null"},
      {"T_e2e_tok_s", r.t_prefill_s + r.t_decode_s > 0
                          ? json_num((n_prompt + n_gen) / (r.t_prefill_s + r.t_decode_s))
                          : "null"},
      {"M_peak_KiB", kib(r.peak)},
      {"M_peak_MiB", mib(r.peak)},
      {"M_rss_after_load_KiB", kib(r.rss_after_load)},
      {"M_rss_after_load_MiB", mib(r.rss_after_load)},
      {"correct", correct < 0 ? "null" : correct ? "true" : "false"},
      {"device", json_str(device_name())},
      {"arch", json_str(arch_name())},
      {"model_sha256", r.sha256.empty() ? "null" : json_str(r.sha256)},
      {"kv_dtype", json_str(c.kv == MYOS_KV_BF16 ? "bf16" : "f32")},
      {"graph", r.graph ? "true" : "false"},
      {"hbm_peak_GBps", json_num(kHbmPeakGBps)},
      {"decode_bytes_per_token", json_num(b_tok)},
      {"achieved_GBps", dev_tok_s > 0 ? json_num(gbps) : "null"},
      {"roofline_frac", dev_tok_s > 0 ? json_num(gbps / kHbmPeakGBps) : "null"},
      {"device_prefill_tok_s", r.dev_prefill_ms > 0 ? json_num(n_prompt / (r.dev_prefill_ms * 1e-3)) : "null"},
      {"device_prefill_ms", json_num(r.dev_prefill_ms)},
      {"device_decode_ms", json_num(r.dev_decode_ms)},
      {"device_decode_tok_s", r.dev_decode_ms > 0 ? json_num(n_gen / (r.dev_decode_ms * 1e-3)) : "null"},
      {"device_weight_bytes", std::to_string(r.weight_bytes)},
      {"device_kv_bytes", std::to_string(r.kv_bytes)},
      {"decode_path", json_str(decode_path_name(r.decode_path))},
      {"M_hwm_KiB", kib(r.hwm)},
      {"verify_mode", verified ? json_str(r.verify_mode) : "null"},
      {"verify_agree", verified ? std::to_string(agree) : "null"},
      {"verify_first_diff", verified && first_diff >= 0 ? std::to_string(first_diff) : "null"},
      {"min_top2_gap", verified && !r.gaps.empty() ? json_num(min_gap) : "null"},
      {"verify_ids", verified ? vids : "null"},
      {"top2_gap_per_step", verified ? gaps : "null"},
      {"timing", json_str("t_load is weight open+parse+upload to HBM and is outside L_prefill and "
                          "T_decode. t_prefill is the prompt prefill (KV and workspace are "
                          "allocated at load) and ends before the first new token. t_decode is "
                          "greedy_decode of n_gen new tokens. device_* are hipEvent times of the "
                          "same two phases. M_peak is the largest VmRSS sample of a 20 ms poll "
                          "from after load to after decode; M_hwm is the kernel's VmHWM. "
                          "roofline_frac = decode_bytes_per_token x device decode tok/s / "
                          "hbm_peak. The verify_* fields come from a second, untimed pass one "
                          "step per call: verify_ids[i] is the greedy id of step i's input "
                          "logits and top2_gap_per_step[i] their top-1 / top-2 gap.")},
  };
  std::string o = "{\n";
  for (size_t i = 0; i < f.size(); i++)
    o += "  \"" + f[i].first + "\": " + f[i].second + (i + 1 < f.size() ? ",\n" : "\n");
  return o + "}\n";
}

}  // namespace

int main(int argc, char **argv) {
  Cli c;
  std::string err;
  if (parse_cli(argc, argv, c, err)) {
    fprintf(stderr, "MyOS: %s\nusage: %s\n", err.c_str(), kUsage);
    return 2;
  }
  std::vector<uint32_t> ref;
  if (c.has_ref && read_token_ids(c.ref_ids, ref, err)) {
    fprintf(stderr, "MyOS ref-ids: %s\n", err.c_str());
    return 1;
  }
  if (!c.block_fixture && !c.has_weights) {
    fprintf(stderr, "MyOS: nothing to decode: pass --weights PATH (or MYOS_WEIGHTS) or --block-fixture\nusage: %s\n", kUsage);
    return 2;
  }
  if (c.arena) {
    // run_arena_cli, main.rs:694-794: this process only spawns and reads
    // children, and never initialises the GPU
    std::vector<uint32_t> prompt;
    if (read_token_ids(c.prompt_ids, prompt, err)) {
      fprintf(stderr, "MyOS prompt-ids: %s\n", err.c_str());
      return 1;
    }
    myos_cli::ArenaJob job;
    char exe[4096];
    const ssize_t n = readlink("/proc/self/exe", exe, sizeof exe - 1);
    if (n <= 0) {
      fprintf(stderr, "MyOS arena: cannot resolve this executable\n");
      return 1;
    }
    exe[n] = '\0';
    job.bin = exe;
    job.weights = c.weights;
    job.prompt_ids = c.prompt_ids;
    job.ref_ids = c.ref_ids;
    job.steps = c.steps;
    job.threads = c.threads;
    job.warmup = c.warmup;
    job.repeats = c.repeats;
    job.out_dir = c.has_fp ? c.fingerprint_dir
                           : "runs/s1-myos-hip-bf16-t" + std::to_string(c.threads);
    if (c.has_shape) job.device_args.push_back(c.shape == MYOS_SHAPE_QWEN25_7B ? "--model-shape=7b" : "--model-shape=1.5b");
    if (c.has_kv) job.device_args.push_back(c.kv == MYOS_KV_BF16 ? "--kv=bf16" : "--kv=f32");
    if (c.has_decode)
      job.device_args.push_back(c.decode == MYOS_DECODE_PERSISTENT ? "--decode-path=persistent"
                                : c.decode == MYOS_DECODE_KERNELS  ? "--decode-path=kernels"
                                : c.decode == MYOS_DECODE_STREAMED ? "--decode-path=streamed"
                                                                   : "--decode-path=auto");
    if (c.no_graph) job.device_args.push_back("--no-graph");
    job.device_args.push_back("--no-hash");
    char hex[65];
    if (myos_sha256_file(c.weights.c_str(), hex) == MYOS_OK) job.model_sha256 = hex;
    return myos_cli::run_arena(job, ref);
  }

  Run r;
  myos_block_shape shape{};
  std::string path = c.weights;
  const bool weights = !c.block_fixture;
  char tmpl[] = "/tmp/myos_fixture_XXXXXX";
  if (c.block_fixture) {
    // the fixture shape (qwen25_block.rs:788-805); --weights with it is only checked
    shape = myos_block_shape{2, 2, 1, 2, 2, 4, 1, 0.0f, 1e6f, 1};
    const int fd = mkstemp(tmpl);
    if (fd < 0) {
      fprintf(stderr, "MyOS Phase1 block fixture failed: cannot create a temporary file\n");
      return 1;
    }
    close(fd);
    path = tmpl;
    if (write_block_fixture(path)) {
      fprintf(stderr, "MyOS Phase1 block fixture failed: cannot write %s\n", path.c_str());
      unlink(tmpl);
      return 1;
    }
    r.prompt = {0};
  } else {
    myos_block_shape_preset(c.shape, &shape);
    if (c.has_prompt) {
      if (read_token_ids(c.prompt_ids, r.prompt, err)) {
        fprintf(stderr, "MyOS prompt-ids: %s\n", err.c_str());
        return 1;
      }
    } else {
      r.prompt = {0};
    }
  }
  r.tokens.assign(c.steps, 0);
  const int rc = decode_timed(path, shape, c, c.has_ref ? &ref : nullptr, r);
  // the weights file is hashed after the run, so that reading it takes no
  // disk or CPU from the load, prefill or decode being timed
  if (rc == 0 && weights && !c.no_hash) {
    char hex[65];
    if (myos_sha256_file(path.c_str(), hex) == MYOS_OK) r.sha256 = hex;
  }
  if (c.block_fixture) unlink(tmpl);
  if (rc) {
    if (c.block_fixture)
      fprintf(stderr, "MyOS Phase1 block fixture failed: %s\n", myos_strerror(rc));
    else
      fprintf(stderr, "MyOS weights %s: %s\n", path.c_str(), myos_strerror(rc));
    return 1;
  }

  const std::string dir = c.has_fp ? c.fingerprint_dir
                                   : std::string("runs/") + (weights ? "s1-weights" : "s1-block-fixture");
  myos_block_shape pinned{};
  myos_block_shape_preset(MYOS_SHAPE_QWEN25_1_5B, &pinned);
  const bool is_pinned = weights && memcmp(&pinned, &shape, sizeof shape) == 0;
  if (write_text(dir, "run_fingerprint.json", fingerprint_json(c, shape, weights, is_pinned, r, argc, argv))) {
    fprintf(stderr, "MyOS fingerprint: cannot write %s/run_fingerprint.json\n", dir.c_str());
    return 1;
  }
  if (weights) {
    if (c.has_prompt) {
      std::string ids;
      for (size_t i = 0; i < r.tokens.size(); i++) ids += (i ? " " : "") + std::to_string(r.tokens[i]);
      if (write_text(dir, "token_ids.txt", ids + "\n")) {
        fprintf(stderr, "MyOS fingerprint: cannot write %s/token_ids.txt\n", dir.c_str());
        return 1;
      }
    }
    const int correct = c.has_ref ? correct_line(r.tokens, ref) == "CORRECT: PASS" : -1;
    if (write_text(dir, "metrics.json", metrics_json(c, shape, r, correct, c.has_ref ? &ref : nullptr))) {
      fprintf(stderr, "MyOS metrics: cannot write %s/metrics.json\n", dir.c_str());
      return 1;
    }
    printf("MyOS Phase1 weights decode (prompt=%u, steps=%zu): %s\n", r.prompt[0], c.steps,
           ids_list(r.tokens).c_str());
  } else {
    printf("MyOS Phase1 block fixture (prompt=0): %s\n", ids_list(r.tokens).c_str());
  }
  if (c.has_ref) printf("%s\n", correct_line(r.tokens, ref).c_str());
  if (c.teacher) {
    // each step fed ref[i]; its greedy id compared with ref[i] (the id the
    // reference chose from the same prefix), with this run's top-2 gap there
    size_t agree = 0;
    long first = -1;
    for (size_t i = 0; i < r.verify_ids.size(); i++) {
      if (i < ref.size() && r.verify_ids[i] == ref[i]) agree++;
      else if (first < 0) first = (long)i;
    }
    if (first < 0)
      printf("TEACHER-FORCED: PASS %zu/%zu\n", agree, r.verify_ids.size());
    else
      printf("TEACHER-FORCED: %zu/%zu first_diff@%ld: got=%u ref=%u gap=%.6g\n", agree,
             r.verify_ids.size(), first, r.verify_ids[first],
             (size_t)first < ref.size() ? ref[first] : 0u, r.gaps[first]);
  }
  return 0;
}
