// Host-only probe of the exported-model reader (csrc/rta_asset.cpp), built by
// tests/test_sanitizers.py with AddressSanitizer and UndefinedBehaviorSanitizer: opens
// one model (and optionally its vocabulary), then asks for every header word, vector,
// matrix and basis the API offers -- in range, at the edges and past them -- and reads
// every byte of what it gets back, so that an out-of-bounds answer shows up as a
// sanitizer report.  Prints one line per call kind; exit 0 unless the sanitizers stop it.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <initializer_list>

#include "../../include/rta.h"

static uint64_t touch(const void* p, uint64_t bytes) {
    const unsigned char* c = static_cast<const unsigned char*>(p);
    uint64_t h = 0;
    for (uint64_t i = 0; i < bytes; ++i) h = h * 31 + c[i];
    return h;
}

int main(int argc, char** argv) {
    if (argc < 2) return 2;
    const char* vocab = (argc > 2 && std::strcmp(argv[2], "-") != 0) ? argv[2] : nullptr;
    char err[256] = {0};
    rta_asset* a = nullptr;
    const int rc = rta_asset_open(argv[1], vocab, &a, err, sizeof err);
    if (rc != RTA_OK) {
        std::printf("open %d %s\n", rc, err);
        return 0;
    }
    rta_asset_info info{};
    std::printf("info %d\n", rta_asset_get_info(a, &info));
    uint64_t words = 0;
    const uint32_t* params = rta_asset_params(a, &words);
    std::printf("params %llu %llx\n", (unsigned long long)words, (unsigned long long)touch(params, words * 4));
    uint64_t h = 0;
    int ok = 0, refused = 0;
    for (int layer = -2; layer <= (int)info.depth; ++layer) {
        for (int field = -1; field <= 64; ++field) {
            uint32_t v = 0;
            if (rta_asset_word(a, layer, field, &v) == RTA_OK) {
                h = h * 31 + v;
                ++ok;
            } else {
                ++refused;
            }
            for (uint64_t count : {(uint64_t)0, (uint64_t)1, (uint64_t)info.hidden, words, ~(uint64_t)0,
                                   ~(uint64_t)0 - 3}) {
                const float* f = nullptr;
                if (rta_asset_vector(a, layer, field, count, &f) == RTA_OK) {
                    h = h * 31 + touch(f, count * 4);
                    ++ok;
                } else {
                    ++refused;
                }
            }
        }
        for (int index = -1; index <= 12; ++index) {
            rta_asset_matrix m{};
            if (rta_asset_layer_matrix(a, layer, index, &m) == RTA_OK) {
                h = h * 31 + touch(m.data, m.avail_bytes);
                ++ok;
            } else {
                ++refused;
            }
        }
    }
    for (int which = -1; which <= 3; ++which) {
        rta_asset_matrix m{};
        if (rta_asset_basis(a, which, &m) == RTA_OK) {
            h = h * 31 + touch(m.data, m.avail_bytes);
            ++ok;
        } else {
            ++refused;
        }
    }
    std::printf("calls ok %d refused %d %llx\n", ok, refused, (unsigned long long)h);
    rta_asset_close(a);
    return 0;
}
