// Host-side sanitizer driver (test infrastructure): runs the PJRT plugin's
// compile pipeline (parse -> inline -> rewrite -> plan, through
// mfx_pjrt_inspect) over StableHLO module texts and over mutated copies of
// them, so AddressSanitizer / UndefinedBehaviorSanitizer see the parser,
// rewriter and planner on malformed input.  No GPU call is made.
//
//   inspect_driver <seed> <mutations per file> <file>...
//
// Exit status 0 when every input was processed (accepted or rejected with an
// error); a sanitizer report aborts the process.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <random>
#include <sstream>
#include <string>
#include <vector>

extern "C" int mfx_pjrt_inspect(const char* text, size_t size, char** json_out);
extern "C" void mfx_pjrt_free(char* p);

namespace {

std::string mutate(const std::string& s, std::mt19937_64& rng) {
  if (s.empty()) return s;
  std::uniform_int_distribution<size_t> pos(0, s.size() - 1);
  std::string t = s;
  switch (rng() % 6) {
    case 0: {  // flip one byte to a printable character or a delimiter
      static const char alphabet[] = "0123456789x<>[](){},:%#@\"\\ -=+.eEabcdfi\n";
      t[pos(rng)] = alphabet[rng() % (sizeof(alphabet) - 1)];
      break;
    }
    case 1: {  // delete a span
      const size_t a = pos(rng), n = 1 + rng() % 64;
      t.erase(a, n);
      break;
    }
    case 2: {  // duplicate a span
      const size_t a = pos(rng), n = 1 + rng() % 64;
      t.insert(a, s.substr(a, n));
      break;
    }
    case 3:  // truncate
      t.resize(pos(rng));
      break;
    case 4: {  // replace a number with an extreme or odd value
      static const char* vals[] = {"0", "-1", "1", "2147483648", "99999999999", "65536", "3", "-0.0", "1e309", "nan"};
      for (int tries = 0; tries < 16; ++tries) {
        const size_t a = pos(rng);
        if (t[a] >= '0' && t[a] <= '9') {
          size_t b = a;
          while (b < t.size() && t[b] >= '0' && t[b] <= '9') ++b;
          size_t c = a;
          while (c > 0 && t[c - 1] >= '0' && t[c - 1] <= '9') --c;
          t.replace(c, b - c, vals[rng() % (sizeof(vals) / sizeof(vals[0]))]);
          break;
        }
      }
      break;
    }
    default: {  // swap two lines (use before definition, reordered ops)
      std::vector<std::string> lines;
      std::istringstream in(s);
      for (std::string l; std::getline(in, l);) lines.push_back(l);
      if (lines.size() > 2) {
        std::uniform_int_distribution<size_t> li(0, lines.size() - 1);
        std::swap(lines[li(rng)], lines[li(rng)]);
      }
      t.clear();
      for (auto& l : lines) t += l + "\n";
    }
  }
  return t;
}

int run(const std::string& text, int& accepted) {
  // The input about to be compiled, for reproducing a sanitizer report.
  if (const char* last = std::getenv("INSPECT_LAST_INPUT")) {
    std::ofstream(last, std::ios::binary | std::ios::trunc) << text;
  }
  char* out = nullptr;
  const int rc = mfx_pjrt_inspect(text.data(), text.size(), &out);
  if (!out) {
    std::fprintf(stderr, "inspect returned no result (rc %d)\n", rc);
    return 1;
  }
  if (rc == 0) ++accepted;
  mfx_pjrt_free(out);
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 4) {
    std::fprintf(stderr, "usage: %s seed mutations file...\n", argv[0]);
    return 2;
  }
  std::mt19937_64 rng(std::strtoull(argv[1], nullptr, 10));
  const int muts = std::atoi(argv[2]);
  int accepted = 0, total = 0;
  for (int i = 3; i < argc; ++i) {
    std::ifstream f(argv[i], std::ios::binary);
    std::stringstream ss;
    ss << f.rdbuf();
    const std::string text = ss.str();
    int acc0 = accepted;
    if (run(text, accepted)) return 1;
    if (accepted == acc0) {
      std::fprintf(stderr, "%s: the unmutated module was rejected\n", argv[i]);
      return 1;
    }
    ++total;
    for (int m = 0; m < muts; ++m, ++total)
      if (run(mutate(text, rng), accepted)) return 1;
  }
  std::printf("inputs %d accepted %d\n", total, accepted);
  return 0;
}
