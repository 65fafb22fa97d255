// gguf_fuzz.cpp — mutation test of the GGUF reader (exactinfer_amd/host/gguf_index.cpp and
// qwen3_schema.cpp), built with AddressSanitizer and UndefinedBehaviorSanitizer by tests/test_gguf.py.
//
// usage: gguf_fuzz <seed file> <iterations> <rng seed> <scratch path> <header bytes>
//
// Each iteration copies the seed file, applies 1-4 mutations (random bytes, a little-endian
// 8- or 4-byte field overwritten with a boundary value, a truncation, a copied span), writes it
// to the scratch path and opens it.  Three mutations in four land in the first <header bytes>
// (the header, metadata and tensor table), the rest anywhere.  A file must either be rejected
// with the reader's FormatError (from the index or from the Qwen3 checks) or be read
// whole: every tensor's bytes are then summed, which touches each view the reader handed out.  Any other exception, a crash
// or a sanitizer report fails the run.  The last line is "ok <accepted> <rejected>".
#include "../../exactinfer_amd/host/gguf_index.h"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

namespace {

struct Rng {  // splitmix64: reproducible from the seed on every platform
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    uint64_t below(uint64_t n) { return n ? next() % n : 0; }
};

size_t g_header = 0;  // bytes before the data section of the seed file

// a position for a field of w bytes: mostly in the header
size_t pick(const std::vector<uint8_t>& b, size_t w, Rng& r) {
    const size_t span = b.size() - w + 1;
    const size_t head = g_header < span ? g_header : span;
    return (r.below(4) != 0 && head > 0) ? r.below(head) : r.below(span);
}

const uint64_t kBoundary[] = {0, 1, 2, 3, 4, 7, 31, 32, 33, 255, 4096, 65535, 1ull << 24, (1ull << 24) + 1,
                              1ull << 26, (1ull << 26) + 1, 100000, 100001, 0x7FFFFFFFull, 0x80000000ull,
                              0xFFFFFFFFull, 1ull << 32, 1ull << 62, 0x7FFFFFFFFFFFFFFFull, 0x8000000000000000ull,
                              0xFFFFFFFFFFFFFFFFull};

void mutate(std::vector<uint8_t>& b, Rng& r) {
    if (b.empty()) return;
    switch (r.below(5)) {
        case 0: {  // a few random bytes
            const uint64_t n = 1 + r.below(4);
            for (uint64_t i = 0; i < n; ++i) b[pick(b, 1, r)] = static_cast<uint8_t>(r.next());
            break;
        }
        case 1:
        case 2: {  // a u64 or u32 field set to a boundary value (counts, lengths, dims, offsets, types)
            const uint64_t v = kBoundary[r.below(sizeof(kBoundary) / sizeof(kBoundary[0]))];
            const size_t w = r.below(2) ? 8 : 4;
            if (b.size() < w) break;
            const size_t at = pick(b, w, r);
            for (size_t i = 0; i < w; ++i) b[at + i] = static_cast<uint8_t>(v >> (8 * i));
            break;
        }
        case 3:  // truncation
            b.resize(pick(b, 1, r));
            break;
        default: {  // a span copied over another place
            const size_t n = 1 + r.below(64);
            if (b.size() <= n) break;
            const size_t from = pick(b, n, r), to = pick(b, n, r);
            for (size_t i = 0; i < n; ++i) b[to + i] = b[from + i];
            break;
        }
    }
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 6) {
        std::fprintf(stderr, "usage: %s seed-file iterations rng-seed scratch-path header-bytes\n", argv[0]);
        return 2;
    }
    std::ifstream in(argv[1], std::ios::binary);
    const std::vector<uint8_t> seed((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
    if (seed.empty()) {
        std::fprintf(stderr, "cannot read %s\n", argv[1]);
        return 2;
    }
    const long iters = std::atol(argv[2]);
    Rng rng{std::strtoull(argv[3], nullptr, 10)};
    const std::string scratch = argv[4];
    g_header = static_cast<size_t>(std::strtoull(argv[5], nullptr, 10));
    long accepted = 0, rejected = 0;
    for (long it = 0; it < iters; ++it) {
        std::vector<uint8_t> b = seed;
        const uint64_t n = 1 + rng.below(4);
        for (uint64_t k = 0; k < n; ++k) mutate(b, rng);
        {
            std::ofstream out(scratch, std::ios::binary | std::ios::trunc);
            out.write(reinterpret_cast<const char*>(b.data()), static_cast<std::streamsize>(b.size()));
        }
        try {
            ei::gguf::Index g(scratch);
            uint64_t sum = 0;
            for (const ei::gguf::TensorSlot& t : g.tensors())
                for (uint64_t i = 0; i < t.bytes; ++i) sum += t.data[i];
            (void)ei::gguf::qwen3_config(g);
            ++accepted;
            if (sum == 1) std::printf(" ");  // keeps the reads
        } catch (const ei::gguf::FormatError&) {
            ++rejected;
        } catch (const std::exception& e) {
            std::fprintf(stderr, "iteration %ld: unexpected exception: %s\n", it, e.what());
            return 1;
        }
    }
    std::printf("ok %ld %ld\n", accepted, rejected);
    return 0;
}
