// Host-only check of the GGUF reader (faie2-flashnext_amd/csrc/gguf.cpp) under AddressSanitizer and
// UndefinedBehaviorSanitizer: parses every file named on the command line; a file the reader accepts has the first
// and last byte of each tensor read back through the mapping.  Built and run by tests/test_gguf_fuzz.py.
#include "../faie2-flashnext_amd/csrc/gguf.h"

#include <cstdio>
#include <string>

namespace fn {
std::string g_fuzz_err;
void set_error(const std::string &m) { g_fuzz_err = m; }
}  // namespace fn

int main(int argc, char **argv) {
    int ok = 0, refused = 0;
    for (int i = 1; i < argc; ++i) {
        fn::Gguf g;
        if (fn::gguf_open(g, argv[i]) != 0) {
            ++refused;
            continue;
        }
        ++ok;
        volatile unsigned s = 0;
        for (const auto &kv : g.tensors)
            if (kv.second.nbytes) s = s + kv.second.data[0] + kv.second.data[kv.second.nbytes - 1];
    }
    std::printf("parsed %d refused %d\n", ok, refused);
    return 0;
}
