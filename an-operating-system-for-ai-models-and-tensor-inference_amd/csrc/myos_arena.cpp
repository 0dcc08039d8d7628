// `myos --arena-s1`: the reference's W/R showdown harness (crates/runtime/
// src/arena.rs:41-75, 92-147, 180-260) for the device build. The parent never
// touches the GPU: it spawns W + R fresh child processes of this binary
// (--weights --prompt-ids --ref-ids --steps --threads --fingerprint-dir
// <out>/warm-i | score-i, plus the device flags), discards the warm-up runs,
// and takes medians over the scored ones (meter.rs:284-317). Gates: DET (all
// scored runs produced identical ids) and CORRECT (DET and the ids equal
// --ref-ids). It writes <out>/metrics.json (medians, min, max, every run),
// det_evidence.json and token_ids.txt. The llama.cpp cost card and verdict
// bands (meter.rs:355-456) compare against a CPU competitor and are not part
// of the device build.
#include "myos_arena.h"

#include <errno.h>
#include <fcntl.h>
#include <spawn.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <sys/wait.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <fstream>
#include <map>
#include <sstream>

extern char **environ;

namespace myos_cli {

namespace {

// A flat JSON object's values: numbers as doubles, strings unescaped,
// true / false / null as the literals (metrics.json is flat).
struct Flat {
  std::map<std::string, std::string> str;
  std::map<std::string, double> num;
  bool has(const std::string &k) const { return num.count(k) != 0; }
};

bool parse_flat(const std::string &t, Flat &out) {
  size_t i = t.find('{');
  if (i == std::string::npos) return false;
  i++;
  auto ws = [&] { while (i < t.size() && isspace((unsigned char)t[i])) i++; };
  auto str = [&](std::string &s) {
    if (t[i] != '"') return false;
    for (i++; i < t.size() && t[i] != '"'; i++) {
      if (t[i] == '\\' && i + 1 < t.size()) i++;
      s += t[i];
    }
    if (i >= t.size()) return false;
    i++;
    return true;
  };
  for (;;) {
    ws();
    if (i >= t.size()) return false;
    if (t[i] == '}') return true;
    if (t[i] == ',') {
      i++;
      continue;
    }
    std::string key;
    if (!str(key)) return false;
    ws();
    if (i >= t.size() || t[i] != ':') return false;
    i++;
    ws();
    if (i >= t.size()) return false;
    if (t[i] == '"') {
      std::string v;
      if (!str(v)) return false;
      out.str[key] = v;
    } else if (t[i] == '[' || t[i] == '{') {
      // nested values are skipped (the harness reads scalars only)
      int depth = 0;
      for (; i < t.size(); i++) {
        if (t[i] == '[' || t[i] == '{') depth++;
        if (t[i] == ']' || t[i] == '}') depth--;
        if (depth == 0) {
          i++;
          break;
        }
      }
    } else {
      size_t j = i;
      while (j < t.size() && t[j] != ',' && t[j] != '}' && !isspace((unsigned char)t[j])) j++;
      const std::string lit = t.substr(i, j - i);
      if (lit == "true" || lit == "false" || lit == "null") out.str[key] = lit;
      else out.num[key] = strtod(lit.c_str(), nullptr);
      i = j;
    }
  }
}

std::string slurp(const std::string &path) {
  std::ifstream f(path);
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
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

std::string num(double v) {
  char b[64];
  snprintf(b, sizeof b, "%.6f", v);
  return b;
}

// median, meter.rs:86-98 (mean of the middle two for an even count)
double median(std::vector<double> v) {
  std::sort(v.begin(), v.end());
  const size_t n = v.size();
  return n % 2 ? v[n / 2] : (v[n / 2 - 1] + v[n / 2]) / 2.0;
}

struct Child {
  Flat metrics;
  std::vector<uint32_t> ids;
  double wall_s = 0;
};

// run_child, arena.rs:92-147: one fresh process, stdout / stderr kept in its
// directory, its metrics.json and token_ids.txt read back and checked
int run_child(const ArenaJob &job, const std::string &dir, Child &c, std::string &err) {
  if (mkdirs(dir)) return err = dir + ": cannot create", -1;
  std::vector<std::string> args = {job.bin,         "--weights",   job.weights,
                                   "--prompt-ids",  job.prompt_ids, "--ref-ids",
                                   job.ref_ids,     "--steps",     std::to_string(job.steps),
                                   "--threads",     std::to_string(job.threads),
                                   "--fingerprint-dir", dir};
  args.insert(args.end(), job.device_args.begin(), job.device_args.end());
  std::vector<char *> argv;
  for (auto &a : args) argv.push_back(const_cast<char *>(a.c_str()));
  argv.push_back(nullptr);
  posix_spawn_file_actions_t fa;
  posix_spawn_file_actions_init(&fa);
  posix_spawn_file_actions_addopen(&fa, 1, (dir + "/stdout.txt").c_str(),
                                   O_WRONLY | O_CREAT | O_TRUNC, 0644);
  posix_spawn_file_actions_addopen(&fa, 2, (dir + "/stderr.txt").c_str(),
                                   O_WRONLY | O_CREAT | O_TRUNC, 0644);
  pid_t pid;
  const auto t0 = std::chrono::steady_clock::now();
  const int sr = posix_spawn(&pid, job.bin.c_str(), &fa, nullptr, argv.data(), environ);
  posix_spawn_file_actions_destroy(&fa);
  if (sr != 0) return err = "spawn " + job.bin + ": " + strerror(sr), -1;
  int status = 0;
  while (waitpid(pid, &status, 0) < 0)
    if (errno != EINTR) return err = "wait for " + dir + ": " + strerror(errno), -1;
  c.wall_s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  std::ofstream(dir + "/wall_s.txt") << num(c.wall_s) << "\n";
  if (!WIFEXITED(status) || WEXITSTATUS(status) != 0) {
    std::string tail = slurp(dir + "/stderr.txt");
    if (tail.size() > 400) tail = tail.substr(tail.size() - 400);
    return err = "child " + dir + " exited " +
                 std::to_string(WIFEXITED(status) ? WEXITSTATUS(status) : 128 + WTERMSIG(status)) +
                 ": " + tail,
           -1;
  }
  if (!parse_flat(slurp(dir + "/metrics.json"), c.metrics))
    return err = dir + "/metrics.json: cannot parse", -1;
  std::ifstream ids(dir + "/token_ids.txt");
  unsigned long long v;
  while (ids >> v) c.ids.push_back((uint32_t)v);
  // check_child_fingerprint, arena.rs:149-178
  const Flat &m = c.metrics;
  if (!m.has("threads") || (size_t)m.num.at("threads") != job.threads)
    return err = dir + ": child threads differ from the requested " + std::to_string(job.threads), -1;
  if (!m.has("batch") || m.num.at("batch") != 1) return err = dir + ": child batch is not 1", -1;
  if (m.str.count("quant_or_dtype") == 0 || m.str.at("quant_or_dtype") != "bf16")
    return err = dir + ": child quant_or_dtype is not bf16", -1;
  if (m.str.count("acc_path") == 0 || m.str.at("acc_path") != "bf16_w_fp32_acc")
    return err = dir + ": child acc_path is not bf16_w_fp32_acc", -1;
  if (!m.has("n_gen") || (size_t)m.num.at("n_gen") != job.steps || c.ids.size() != job.steps)
    return err = dir + ": child n_gen / token_ids differ from --steps", -1;
  if (!m.has("M_peak_MiB")) return err = dir + ": M_peak is missing", -1;
  return 0;
}

// the phase figures the medians are taken over, meter.rs:48-78 / 284-317,
// plus the device ones
const char *kFields[] = {"T_decode_tok_s", "L_TTFT_ms",  "L_TPOT_ms", "M_peak_MiB",
                         "T_e2e_tok_s",    "t_load_s",   "device_decode_tok_s",
                         "device_prefill_ms", "device_decode_ms", "roofline_frac"};

std::string runs_json(const std::vector<Child> &runs) {
  std::string o = "[";
  for (size_t r = 0; r < runs.size(); r++) {
    o += r ? ", {" : "{";
    bool first = true;
    for (const char *k : kFields)
      if (runs[r].metrics.has(k)) {
        o += std::string(first ? "" : ", ") + "\"" + k + "\": " + num(runs[r].metrics.num.at(k));
        first = false;
      }
    o += std::string(first ? "" : ", ") + "\"wall_s\": " + num(runs[r].wall_s) + "}";
  }
  return o + "]";
}

std::string stat_json(const std::vector<Child> &runs, int which) {
  // which: 0 median, 1 min, 2 max
  std::string o = "{";
  bool first = true;
  for (const char *k : kFields) {
    std::vector<double> v;
    for (auto &c : runs)
      if (c.metrics.has(k)) v.push_back(c.metrics.num.at(k));
    if (v.size() != runs.size() || v.empty()) continue;
    const double x = which == 0 ? median(v)
                                : which == 1 ? *std::min_element(v.begin(), v.end())
                                             : *std::max_element(v.begin(), v.end());
    o += std::string(first ? "" : ", ") + "\"" + k + "\": " + num(x);
    first = false;
  }
  return o + "}";
}

std::string ids_str(const std::vector<uint32_t> &ids, const char *sep) {
  std::string s;
  for (size_t i = 0; i < ids.size(); i++) s += (i ? sep : "") + std::to_string(ids[i]);
  return s;
}

}  // namespace

int run_arena(const ArenaJob &job, const std::vector<uint32_t> &ref) {
  if (mkdirs(job.out_dir)) {
    fprintf(stderr, "MyOS arena: %s: cannot create\n", job.out_dir.c_str());
    return 1;
  }
  std::vector<Child> warm(job.warmup), score(job.repeats);
  std::string err;
  for (size_t i = 0; i < job.warmup; i++) {
    fprintf(stderr, "=== WARM %zu/%zu ===\n", i + 1, job.warmup);
    if (run_child(job, job.out_dir + "/warm-" + std::to_string(i + 1), warm[i], err)) {
      fprintf(stderr, "MyOS arena: %s\n", err.c_str());
      return 1;
    }
  }
  for (size_t i = 0; i < job.repeats; i++) {
    fprintf(stderr, "=== SCORE %zu/%zu ===\n", i + 1, job.repeats);
    if (run_child(job, job.out_dir + "/score-" + std::to_string(i + 1), score[i], err)) {
      fprintf(stderr, "MyOS arena: %s\n", err.c_str());
      return 1;
    }
  }
  // summarize, arena.rs:180-260
  bool det = true;
  for (auto &c : score) det = det && c.ids == score[0].ids && c.ids.size() == job.steps;
  const bool correct = det && score[0].ids == ref;
  bool warm_match = true;
  for (auto &c : warm) warm_match = warm_match && c.ids == score[0].ids;
  const Flat &m0 = score[0].metrics;
  auto s = [&](const char *k) {
    return m0.str.count(k) ? "\"" + m0.str.at(k) + "\"" : std::string("null");
  };
  std::string o = "{\n";
  o += "  \"scenario_id\": \"S1\",\n  \"impl\": \"myos-hip\",\n";
  o += "  \"quant_or_dtype\": \"bf16\",\n  \"acc_path\": \"bf16_w_fp32_acc\",\n";
  o += "  \"threads\": " + std::to_string(job.threads) + ",\n  \"batch\": 1,\n";
  o += "  \"n_prompt\": " + num(m0.has("n_prompt") ? m0.num.at("n_prompt") : 0) + ",\n";
  o += "  \"n_gen\": " + std::to_string(job.steps) + ",\n";
  o += "  \"W\": " + std::to_string(job.warmup) + ",\n  \"R\": " + std::to_string(job.repeats) + ",\n";
  o += std::string("  \"det\": \"") + (det ? "PASS" : "FAIL") + "\",\n";
  o += std::string("  \"CORRECT\": \"") + (correct ? "PASS" : "FAIL") + "\",\n";
  o += std::string("  \"warmup_ids_match_scored\": ") + (warm_match ? "true" : "false") + ",\n";
  o += "  \"device\": " + s("device") + ",\n  \"arch\": " + s("arch") + ",\n";
  o += "  \"decode_path\": " + s("decode_path") + ",\n  \"kv_dtype\": " + s("kv_dtype") + ",\n";
  o += "  \"model_sha256\": " + (job.model_sha256.empty() ? std::string("null") : "\"" + job.model_sha256 + "\"") + ",\n";
  o += "  \"median\": " + stat_json(score, 0) + ",\n";
  o += "  \"min\": " + stat_json(score, 1) + ",\n";
  o += "  \"max\": " + stat_json(score, 2) + ",\n";
  o += "  \"per_run_scored\": " + runs_json(score) + ",\n";
  o += "  \"per_run_warmup_discarded\": " + runs_json(warm) + ",\n";
  o += "  \"note\": \"Each run is a fresh process of this binary (score-i / warm-i hold its "
       "metrics.json, token_ids.txt, stdout and stderr). Medians over the scored runs; warm-up "
       "runs are discarded. The llama.cpp cost card of the reference's arena is not produced.\"\n";
  o += "}\n";
  std::ofstream(job.out_dir + "/metrics.json") << o;
  std::string d = "{\n";
  d += std::string("  \"det\": \"") + (det ? "PASS" : "FAIL") + "\",\n";
  d += std::string("  \"CORRECT\": \"") + (correct ? "PASS" : "FAIL") + "\",\n";
  d += "  \"scored_ids\": [";
  for (size_t i = 0; i < score.size(); i++) d += (i ? ", [" : "[") + ids_str(score[i].ids, ", ") + "]";
  d += "],\n  \"warmup_ids\": [";
  for (size_t i = 0; i < warm.size(); i++) d += (i ? ", [" : "[") + ids_str(warm[i].ids, ", ") + "]";
  d += "],\n  \"ref_ids\": [" + ids_str(ref, ", ") + "]\n}\n";
  std::ofstream(job.out_dir + "/det_evidence.json") << d;
  std::ofstream(job.out_dir + "/token_ids.txt") << ids_str(score[0].ids, " ") << "\n";
  std::vector<double> v[4];
  const char *keys[4] = {"T_decode_tok_s", "L_TTFT_ms", "L_TPOT_ms", "M_peak_MiB"};
  for (int k = 0; k < 4; k++)
    for (auto &c : score) v[k].push_back(c.metrics.has(keys[k]) ? c.metrics.num.at(keys[k]) : NAN);
  printf("ARENA S1 threads=%zu W=%zu R=%zu CORRECT=%s DET=%s T_decode=%.4f L_TTFT_ms=%.3f "
         "L_TPOT_ms=%.3f M_peak_MiB=%.3f\n",
         job.threads, job.warmup, job.repeats, correct ? "PASS" : "FAIL", det ? "PASS" : "FAIL",
         median(v[0]), median(v[1]), median(v[2]), median(v[3]));
  printf("run-dir: %s\n", job.out_dir.c_str());
  return correct && det ? 0 : 1;
}

}  // namespace myos_cli
