// The W/R showdown harness of the `myos` CLI (crates/runtime/src/arena.rs).
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

namespace myos_cli {

struct ArenaJob {
  std::string bin;                       // this executable
  std::string weights, prompt_ids, ref_ids, out_dir;
  size_t steps = 128, threads = 8, warmup = 3, repeats = 5;
  std::vector<std::string> device_args;  // --model-shape / --kv / --decode-path passed on
  std::string model_sha256;              // hashed once by the parent (empty: unreadable)
};

// Runs W warm-up + R scored child processes, writes the aggregate files and
// prints the ARENA line; returns the process exit code (0 when DET and
// CORRECT pass).
int run_arena(const ArenaJob &job, const std::vector<uint32_t> &ref);

}  // namespace myos_cli
