// st_parse_fuzz.cpp -- CPU fuzz driver for the safetensors header parser
// (fastmlx_amd/csrc/fmx_st_parse.cpp).  Test infrastructure: tests/
// test_host_sanitize.py builds it with AddressSanitizer and UndefinedBehavior-
// Sanitizer and runs it on the reference fixture's blobs.
//
// Each seed (a valid safetensors blob) is mutated many times: byte overwrites,
// truncations, a rewritten 8-byte header length, JSON tokens spliced into the
// header, and repeated ranges.  Every mutant is parsed; an accepted one is
// walked through the accessors, and every tensor range must lie in the blob.  A
// memory error, undefined behaviour or a broken invariant ends the run with a
// nonzero status.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/fmx.h"

namespace {

uint64_t rng_state = 0x9E3779B97F4A7C15ull;
uint64_t rnd() {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return rng_state;
}
size_t pick(size_t n) { return n ? (size_t)(rnd() % n) : 0; }

const char* kTokens[] = {"{", "}", "[", "]", ",", ":", "\"", "\\", "\\u", "\\ud800", "\\udc00",
                         "\\u0000", "1e99", "-", "-1", "0", "18446744073709551615",
                         "99999999999999999999", "null", "true", "false", "\"dtype\"", "\"shape\"",
                         "\"data_offsets\"", "\"__metadata__\"", "\"F32\"", "\"BF16\"", "\"U8\"",
                         "\"XYZ\"", "[0,0]", "[1,2,3]", "{}", "[]", "\"w\"", " ", "\n", "\x7f",
                         "\xff", "\xc3\xa9"};

void check(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "invariant broken: %s\n", what);
    std::abort();
  }
}

// Parse one blob; on success walk every accessor and check the ranges.
bool parse_and_walk(const std::vector<uint8_t>& b) {
  fmx_st_header* h = nullptr;
  const int rc = fmx_safetensors_parse(b.data(), b.size(), &h);
  if (rc != 0) {
    check(h == nullptr, "failed parse leaves the result null");
    return false;
  }
  check(h != nullptr, "successful parse returns a header");
  const uint64_t ds = fmx_safetensors_data_start(h);
  check(ds == 8 + fmx_safetensors_header_size(h) && ds <= b.size(), "data start inside the blob");
  const int64_t n = fmx_safetensors_count(h);
  for (int64_t i = 0; i < n; ++i) {
    const char *name = nullptr, *dtype = nullptr;
    int ndim = -1;
    const int64_t* shape = nullptr;
    uint64_t beg = 0, end = 0, off = 0;
    check(fmx_safetensors_tensor(h, i, &name, &dtype, &ndim, &shape, &beg, &end) == 0, "tensor");
    check(name && dtype && ndim >= 0 && beg <= end, "tensor fields");
    for (int d = 0; d < ndim; ++d) check(shape[d] >= 0, "non-negative axis");
    check(fmx_safetensors_slice(b.size(), ds, beg, end, &off) == 0 && off + (end - beg) <= b.size(),
          "tensor range inside the blob");
    const int64_t j = fmx_safetensors_find(h, name);
    const char* jn = nullptr;
    check(j >= 0 && fmx_safetensors_tensor(h, j, &jn, nullptr, nullptr, nullptr, nullptr,
                                           nullptr) == 0 && std::strcmp(jn, name) == 0,
          "find returns the named tensor");
    fmx_dtype dt;
    (void)fmx_safetensors_dtype(dtype, &dt);
  }
  check(fmx_safetensors_tensor(h, n, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr) != 0,
        "index past the end is refused");
  const int64_t nm = fmx_safetensors_metadata_count(h);
  for (int64_t i = 0; i < nm; ++i) {
    const char *k = nullptr, *v = nullptr;
    check(fmx_safetensors_metadata(h, i, &k, &v) == 0 && k && v, "metadata entry");
  }
  fmx_safetensors_free(h);
  return true;
}

std::vector<uint8_t> mutate(const std::vector<uint8_t>& seed) {
  std::vector<uint8_t> b = seed;
  const int rounds = 1 + (int)pick(4);
  for (int r = 0; r < rounds; ++r) {
    uint64_t hlen = 0;
    if (b.size() >= 8) std::memcpy(&hlen, b.data(), 8);
    const size_t hend = (size_t)(8 + (hlen < b.size() ? hlen : 0));
    switch (pick(6)) {
      case 0:  // overwrite a few bytes
        for (int k = 0, nk = 1 + (int)pick(8); k < nk && !b.empty(); ++k) b[pick(b.size())] = (uint8_t)rnd();
        break;
      case 1:  // truncate
        b.resize(pick(b.size() + 1));
        break;
      case 2: {  // rewrite the header length
        const uint64_t choices[] = {0, 1, 2, hlen + 1, hlen - 1, (uint64_t)b.size(),
                                    (uint64_t)b.size() - 7, ~0ull, 1ull << 63, rnd()};
        const uint64_t v = choices[pick(sizeof(choices) / sizeof(choices[0]))];
        if (b.size() >= 8) std::memcpy(b.data(), &v, 8);
        break;
      }
      case 3: {  // splice a JSON token into the header
        const std::string tok = kTokens[pick(sizeof(kTokens) / sizeof(kTokens[0]))];
        const size_t at = 8 + pick(hend > 8 ? hend - 8 : 1);
        if (at <= b.size()) b.insert(b.begin() + (long)at, tok.begin(), tok.end());
        break;
      }
      case 4: {  // delete a range
        if (b.size() > 9) {
          const size_t at = 8 + pick(b.size() - 8), n = 1 + pick(16);
          b.erase(b.begin() + (long)at, b.begin() + (long)(at + n < b.size() ? at + n : b.size()));
        }
        break;
      }
      default: {  // repeat a range
        if (b.size() > 9) {
          const size_t at = 8 + pick(b.size() - 8), n = 1 + pick(32);
          const size_t e = at + n < b.size() ? at + n : b.size();
          std::vector<uint8_t> piece(b.begin() + (long)at, b.begin() + (long)e);
          b.insert(b.begin() + (long)at, piece.begin(), piece.end());
        }
        break;
      }
    }
  }
  return b;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 3) {
    std::fprintf(stderr, "usage: %s ITERATIONS SEED_FILE...\n", argv[0]);
    return 2;
  }
  const long iters = std::atol(argv[1]);
  long accepted = 0, total = 0;
  for (int f = 2; f < argc; ++f) {
    FILE* fp = std::fopen(argv[f], "rb");
    if (!fp) return 2;
    std::vector<uint8_t> seed;
    for (int c; (c = std::fgetc(fp)) != EOF;) seed.push_back((uint8_t)c);
    std::fclose(fp);
    check(parse_and_walk(seed), "the seed itself parses");
    for (long i = 0; i < iters; ++i, ++total) accepted += parse_and_walk(mutate(seed));
  }
  // Blobs of random bytes and random lengths.
  for (long i = 0; i < iters; ++i, ++total) {
    std::vector<uint8_t> b(pick(300));
    for (auto& v : b) v = (uint8_t)rnd();
    accepted += parse_and_walk(b);
  }
  std::printf("%ld mutants parsed, %ld accepted\n", total, accepted);
  return 0;
}
