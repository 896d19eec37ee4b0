// CPU test of the staged boundary copies' host side (camel_hip::for_each_chunk
// and camel_hip::CopyPool from camel_amd/csrc/hip/host_copy.h): chunk plans
// at slot edges, and parallel copies of every size class from unaligned
// sources into unaligned destinations, byte for byte.  Built with g++ (and
// with -fsanitize=thread) by tests/test_host_copy.py.
#include "host_copy.h"

#include <cstdio>
#include <random>
#include <vector>

using namespace camel_hip;

static int failures = 0;
#define EXPECT(c)                                                                                  \
    do {                                                                                           \
        if (!(c)) {                                                                                \
            std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c);                                \
            ++failures;                                                                            \
        }                                                                                          \
    } while (0)

static void check_plan(size_t bytes, size_t slot) {
    size_t next = 0, count = 0, expect_index = 0;
    for_each_chunk(bytes, slot, [&](size_t i, size_t off, size_t m) {
        EXPECT(i == expect_index++);
        EXPECT(off == next);
        EXPECT(m > 0 && m <= slot);
        // every chunk but the last is a whole slot
        EXPECT(off + m == bytes || m == slot);
        next = off + m;
        ++count;
    });
    EXPECT(next == bytes);
    EXPECT(count == (bytes + slot - 1) / slot);
}

int main() {
    const size_t slot = size_t(8) << 20;
    for (size_t b : {size_t(0), size_t(1), size_t(1) << 20, (size_t(2) << 20) - 1, size_t(2) << 20,
                     slot - 1, slot, slot + 1, 2 * slot, 3 * slot - 1, 3 * slot + 5,
                     7 * slot + 4093, size_t(67108864), size_t(201326592)})
        check_plan(b, slot);

    // piece boundaries: ascending, 4 KiB aligned, covering [0, n)
    CopyPool probe(3);
    for (size_t n : {size_t(1) << 20, (size_t(1) << 20) + 1, (size_t(4) << 20) - 7, slot,
                     slot - 1, slot + 12345}) {
        const int parts = probe.pieces(n);
        EXPECT(parts >= 1 && parts <= 4);
        size_t prev = 0;
        for (int p = 0; p <= parts; ++p) {
            const size_t a = CopyPool::begin(n, parts, p);
            EXPECT(a >= prev && a <= n);
            if (p > 0 && p < parts) EXPECT(a % 4096 == 0);
            prev = a;
        }
        EXPECT(CopyPool::begin(n, parts, 0) == 0 && CopyPool::begin(n, parts, parts) == n);
    }

    // copies: sizes around the piece and slot edges, source and destination
    // at every offset mod 8 (the reference's payload is 8-byte aligned only)
    std::mt19937_64 rng(7);
    const size_t cap = slot + 64;
    std::vector<unsigned char> src(cap + 16), dst(cap + 16);
    for (auto &c : src) c = (unsigned char)rng();
    CopyPool pool(3);
    size_t cases = 0;
    for (size_t n : {size_t(0), size_t(1), size_t(4095), (size_t(1) << 20) - 1, size_t(1) << 20,
                     (size_t(2) << 20) + 3, (size_t(4) << 20) + 4097, slot - 1, slot}) {
        for (size_t so : {0, 1, 3, 8}) {
            for (size_t d_o : {0, 5, 8}) {
                std::fill(dst.begin(), dst.end(), 0xA5);
                pool.copy(dst.data() + d_o, src.data() + so, n);
                EXPECT(std::memcmp(dst.data() + d_o, src.data() + so, n) == 0);
                for (size_t i = 0; i < d_o; ++i) EXPECT(dst[i] == 0xA5);
                EXPECT(dst[d_o + n] == 0xA5); // nothing written past the end
                ++cases;
            }
        }
    }
    // many copies in a row through one pool (the workers' generations)
    for (int r = 0; r < 200; ++r) {
        const size_t n = (size_t(1) << 20) * (1 + r % 5) + (size_t)(r * 977 % 4096);
        pool.copy(dst.data() + (r & 7), src.data() + ((r >> 3) & 7), n);
        EXPECT(std::memcmp(dst.data() + (r & 7), src.data() + ((r >> 3) & 7), n) == 0);
        ++cases;
    }
    std::printf("cases=%zu failures=%d\n", cases, failures);
    return failures == 0 ? 0 : 1;
}
