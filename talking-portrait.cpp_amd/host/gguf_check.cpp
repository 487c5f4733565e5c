// gguf_check: open a GGUF file with the library's reader and read tensors,
// for running the reader under AddressSanitizer / UndefinedBehaviorSanitizer
// (host/Makefile.sanitize) on well-formed and malformed files.
//
//   gguf_check FILE [ARCH|-] [TENSOR ...]
//
// Reads every tensor named (every tensor of the file when none is named) and
// prints "ok <name> <elements> <f16> <sum>" per tensor, or "error: <message>"
// and exits 1 at the first failure, as the library's entry points report it.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "gguf.h"

int main(int argc, char **argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s FILE [ARCH|-] [TENSOR ...]\n", argv[0]);
        return 2;
    }
    const char *arch = argc > 2 && strcmp(argv[2], "-") != 0 ? argv[2] : nullptr;
    tp::gguf_file f;
    std::string err;
    if (!f.open(argv[1], arch, err)) {
        printf("error: %s\n", err.c_str());
        return 1;
    }
    std::vector<std::string> names;
    for (int i = 3; i < argc; i++) names.push_back(argv[i]);
    if (names.empty())
        for (const auto &t : f.tensors) names.push_back(t.name);
    std::vector<float> v;
    for (const auto &n : names) {
        bool f16 = false;
        if (!f.read(n, v, f16, err)) {
            printf("error: %s\n", err.c_str());
            return 1;
        }
        double sum = 0;
        for (float x : v) sum += x;
        printf("ok %s %zu %d %.9g\n", n.c_str(), v.size(), f16 ? 1 : 0, sum);
    }
    return 0;
}
