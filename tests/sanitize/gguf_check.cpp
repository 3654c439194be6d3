// Sanitizer driver for the host GGUF reader (fuel_amd/csrc/gguf.cpp): opens
// every file named on the command line with frq::gguf::open, walks all
// metadata values and tensor records, and prints one line per file (the parse
// error, or counts and a checksum).  Built with -fsanitize=address,undefined
// by tests/sanitize/run.sh and run over well-formed, truncated and corrupted
// files; any sanitizer report fails the run.
#include <stdio.h>

#include <string>

#include "../../fuel_amd/csrc/gguf.hpp"

namespace {

unsigned long long walk(const frq::gguf::Value& v) {
    unsigned long long h = (unsigned long long)v.type * 1000003ull + v.u + (unsigned long long)v.i;
    h += (unsigned long long)(v.f * 1024.0);
    for (unsigned char c : v.s) h = h * 131 + c;
    for (const auto& e : v.a) h = h * 31 + walk(e);
    return h;
}

}  // namespace

int main(int argc, char** argv) {
    for (int i = 1; i < argc; i++) {
        std::string err;
        auto f = frq::gguf::open(argv[i], err);
        if (!f) {
            printf("%s: error: %s\n", argv[i], err.c_str());
            continue;
        }
        unsigned long long h = (unsigned long long)f->version;
        for (const auto& kv : f->metadata) {
            for (unsigned char c : kv.first) h = h * 131 + c;
            h = h * 31 + walk(kv.second);
        }
        unsigned long long last = 0;
        for (const auto& t : f->tensors) {
            for (uint64_t d : t.dims) h = h * 31 + d;
            h = h * 31 + t.offset + t.nbytes + (unsigned long long)t.ggml_dtype;
            // touch the tensor's last byte when it lies inside the map
            const uint64_t end = f->tensor_data_offset + t.offset + t.nbytes;
            if (t.nbytes && end <= f->map_bytes) last += f->map[end - 1];
        }
        printf("%s: v%d %zu meta %zu tensors data@%llu hash %llx %llu\n", argv[i], f->version, f->metadata.size(),
               f->tensors.size(), (unsigned long long)f->tensor_data_offset, h, last);
    }
    return 0;
}
