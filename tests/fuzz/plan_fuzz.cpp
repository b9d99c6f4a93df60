// Host-only fuzz harness for the tensor-plan reader, validator and fuser
// (browsergrad_amd/csrc/plan.cpp, plan_fuse.cpp), built with AddressSanitizer
// and UndefinedBehaviorSanitizer by the Makefile beside it.
//
// Every seed plan given on the command line (a JSON file; an optional second
// file of the same name plus ".req" is its semantic side table) is run
// through bg::inspect_plan as is and then under a fixed number of seeded
// mutations: byte flips, truncations, spliced duplicates, numeric
// perturbations and token swaps.  Malformed input must come back as a
// bg::Error (a refusal), never as a sanitizer report, crash or hang.  The
// runtime entry points the executor would call are absent from this build:
// inspect_plan parses, validates and fuses without running anything.
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <random>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../browsergrad_amd/csrc/core.h"

namespace bg {
[[noreturn]] void fail(int code, const std::string& msg) { throw Error(code, msg); }
int64_t numel(const std::vector<int64_t>& shape) {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  return n;
}
[[noreturn]] static void absent() { fail(BG_E_UNSUPPORTED, "runtime call in the host-only fuzz build"); }
Profile::Profile(bg_ctx*, const char*, int64_t, int64_t) { absent(); }
Profile::~Profile() {}
Record& get(bg_ctx*, bg_handle, const char*) { absent(); }
bg_handle mint(bg_ctx*, size_t, const std::vector<int64_t>&, int) { absent(); }
void launch_optimizer_fused(bg_ctx*, int, const bg_optim_args&, double, double, double, double,
                            const float* const (&)[4], float*, int64_t) {
  absent();
}
void launch_reduce_lead(bg_ctx*, const void*, int, int64_t, int64_t, int64_t, int, void*, int) { absent(); }
int64_t dtype_size(int) { absent(); }
}  // namespace bg

extern "C" {
#define BG_ABSENT(name, ...) \
  int name(__VA_ARGS__) { return BG_E_UNSUPPORTED; }
BG_ABSENT(bg_attention_ex, bg_ctx*, const bg_attention_desc*, bg_handle*)
BG_ABSENT(bg_cast, bg_ctx*, bg_handle, int, int, const int64_t*, int, bg_handle*)
BG_ABSENT(bg_conv_ex, bg_ctx*, const bg_conv_desc*, bg_handle*)
BG_ABSENT(bg_copy_strided, bg_ctx*, bg_handle, int64_t, const int64_t*, const int64_t*, int, bg_handle*)
BG_ABSENT(bg_fused_ex, bg_ctx*, const bg_fused_desc*, bg_handle*)
BG_ABSENT(bg_layer_norm, bg_ctx*, bg_handle, bg_handle, bg_handle, int64_t, int64_t, float, int, bg_handle*)
BG_ABSENT(bg_layer_norm_backward_bias, bg_ctx*, bg_handle, int64_t, int64_t, bg_handle*)
BG_ABSENT(bg_layer_norm_backward_input, bg_ctx*, bg_handle, bg_handle, bg_handle, int64_t, int64_t, float,
          bg_handle*)
BG_ABSENT(bg_layer_norm_backward_weight, bg_ctx*, bg_handle, bg_handle, int64_t, int64_t, float, bg_handle*)
BG_ABSENT(bg_matmul_ex, bg_ctx*, const bg_matmul_desc*, bg_handle*)
BG_ABSENT(bg_matmul_ex2, bg_ctx*, const bg_matmul_desc*, const bg_matmul_ext*, bg_handle*)
BG_ABSENT(bg_optimizer_update, bg_ctx*, int, const bg_handle*, int, const bg_optim_args*, int64_t, bg_handle*)
BG_ABSENT(bg_reduce_last, bg_ctx*, bg_handle, int64_t, int64_t, int, int, bg_handle*)
BG_ABSENT(bg_release, bg_ctx*, bg_handle)
BG_ABSENT(bg_reshape, bg_ctx*, bg_handle, const int64_t*, int, bg_handle*)
BG_ABSENT(bg_softmax_last, bg_ctx*, bg_handle, int64_t, int64_t, int, bg_handle*)
BG_ABSENT(bg_upload, bg_ctx*, const void*, size_t, const int64_t*, int, int, bg_handle*)
}

static std::string slurp(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

static std::string mutate(const std::string& s, std::mt19937_64& rng) {
  std::string m = s;
  if (m.empty()) return m;
  std::uniform_int_distribution<size_t> pos(0, m.size() - 1);
  switch (rng() % 6) {
    case 0:  // flip a byte
      m[pos(rng)] = char(rng() & 0xff);
      break;
    case 1:  // truncate
      m.resize(pos(rng));
      break;
    case 2: {  // splice a copy of a span elsewhere
      const size_t a = pos(rng), b = pos(rng), at = pos(rng);
      m.insert(at, m.substr(std::min(a, b), (std::max(a, b) - std::min(a, b)) % 512));
      break;
    }
    case 3: {  // perturb a number: the next digit run becomes a large, negative or huge value
      const size_t at = m.find_first_of("0123456789", pos(rng));
      if (at == std::string::npos) break;
      const size_t end = m.find_first_not_of("0123456789", at);
      static const char* repl[] = {"-1", "0", "99999999999999999999", "4294967296", "1e308", "-9223372036854775808",
                                   "2147483648", "8", "7"};
      m.replace(at, (end == std::string::npos ? m.size() : end) - at, repl[rng() % 9]);
      break;
    }
    case 4: {  // swap one JSON token for another
      static const char* tok[] = {"null", "true", "[]", "{}", "\"\"", "\"CAST\"", "\"+PROGRAM\"", "-Infinity",
                                  "[[0,1,1]]", "\"float64\""};
      const size_t at = pos(rng);
      m.replace(at, std::min<size_t>(rng() % 8, m.size() - at), tok[rng() % 10]);
      break;
    }
    default: {  // delete a span
      const size_t at = pos(rng);
      m.erase(at, std::min<size_t>(1 + rng() % 32, m.size() - at));
    }
  }
  return m;
}

int main(int argc, char** argv) {
  if (argc < 3) {
    std::fprintf(stderr, "usage: %s <mutations per seed> <seed.json>...\n", argv[0]);
    return 2;
  }
  const long per_seed = std::atol(argv[1]);
  std::mt19937_64 rng(20261202);
  long accepted = 0, refused = 0;
  for (int i = 2; i < argc; ++i) {
    const std::string plan = slurp(argv[i]);
    std::string req;
    {
      std::ifstream rf(std::string(argv[i]) + ".req", std::ios::binary);
      if (rf) {
        std::stringstream ss;
        ss << rf.rdbuf();
        req = ss.str();
      }
    }
    for (long k = -1; k < per_seed; ++k) {
      const std::string p = k < 0 ? plan : mutate(plan, rng);
      const std::string r = req.empty() || k < 0 || rng() % 2 ? req : mutate(req, rng);
      try {
        bg::inspect_plan(p.c_str(), r.empty() ? nullptr : r.c_str());
        ++accepted;
      } catch (const bg::Error& e) {
        ++refused;
        if (k < 0) {
          std::fprintf(stderr, "seed %s was refused unmutated: %s\n", argv[i], e.what());
          return 1;
        }
      }
    }
  }
  std::printf("plan_fuzz: %ld accepted, %ld refused, no sanitizer report\n", accepted, refused);
  return 0;
}
