// Parses every file named on the command line with the GGUF reader
// (nspeech_amd/host/gguf.cpp, built into this program with AddressSanitizer)
// and prints "ok <path>" or "err <path>": malformed inputs must end in an
// error, never in an out-of-bounds access (which ASan aborts on).
#include <cstdio>
#include <fstream>
#include <iterator>
#include <vector>

#include "gguf.h"

int main(int argc, char** argv) {
  for (int i = 1; i < argc; ++i) {
    std::ifstream f(argv[i], std::ios::binary);
    std::vector<char> img((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    // an exact-size heap copy, so a read one byte past the end is caught
    std::vector<uint8_t> buf(img.begin(), img.end());
    uint8_t* p = buf.empty() ? nullptr : new uint8_t[buf.size()];
    if (p) std::copy(buf.begin(), buf.end(), p);
    try {
      auto c = nspeech::rocm::gguf::Content::read(p, buf.size());
      size_t sum = 0;
      for (const auto& t : c.tensor_infos()) {
        const uint8_t* d = c.tensor_data(t);
        for (uint64_t k = 0; k < t.nbytes; ++k) sum += d[k];
      }
      std::printf("ok %s %zu\n", argv[i], sum);
    } catch (const std::exception& e) {
      std::printf("err %s\n", argv[i]);
    }
    delete[] p;
  }
  return 0;
}
