// sha256.hpp -- SHA-256 (FIPS 180-4) for the packed checkpoint's file
// digests. The reference hashes with the `sha2` crate (export_packed.rs:4,
// :60-70) and Python's hashlib (prepare_hf_q4.py:31-36); this is the
// standard's algorithm written out: 64-byte blocks, the 64-entry message
// schedule, eight working variables, big-endian length padding.
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

namespace decisive {

class Sha256 {
public:
    Sha256() { reset(); }

    void reset() {
        static const uint32_t init[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                         0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
        memcpy(h_, init, sizeof h_);
        length_ = 0;
        fill_ = 0;
    }

    void update(const void *data, size_t n) {
        const uint8_t *p = (const uint8_t *)data;
        length_ += n;
        if (fill_) {
            size_t take = n < 64 - fill_ ? n : 64 - fill_;
            memcpy(block_ + fill_, p, take);
            fill_ += take;
            p += take;
            n -= take;
            if (fill_ < 64) return;
            compress(block_);
            fill_ = 0;
        }
        for (; n >= 64; p += 64, n -= 64) compress(p);
        memcpy(block_, p, n);
        fill_ = n;
    }

    // The digest as 64 lowercase hex characters; the object is reset after.
    std::string hex() {
        uint8_t pad[72] = {0x80};
        const uint64_t bits = length_ * 8;
        const size_t zeros = (fill_ < 56 ? 56 - fill_ : 120 - fill_);
        uint8_t len[8];
        for (int i = 0; i < 8; i++) len[i] = (uint8_t)(bits >> (56 - 8 * i));
        update(pad, zeros);
        update(len, 8);
        std::string out;
        char buf[9];
        for (uint32_t v : h_) {
            snprintf(buf, sizeof buf, "%08x", v);
            out += buf;
        }
        reset();
        return out;
    }

    static std::string of(const void *data, size_t n) {
        Sha256 s;
        s.update(data, n);
        return s.hex();
    }

private:
    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

    void compress(const uint8_t *b) {
        static const uint32_t k[64] = {
            0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
            0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
            0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
            0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
            0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
            0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
            0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
            0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
        uint32_t w[64];
        for (int i = 0; i < 16; i++)
            w[i] = (uint32_t)b[4 * i] << 24 | (uint32_t)b[4 * i + 1] << 16 | (uint32_t)b[4 * i + 2] << 8 | b[4 * i + 3];
        for (int i = 16; i < 64; i++) {
            uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h_[0], bb = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], h = h_[7];
        for (int i = 0; i < 64; i++) {
            uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[i] + w[i];
            uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & bb) ^ (a & c) ^ (bb & c));
            h = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = bb;
            bb = a;
            a = t1 + t2;
        }
        h_[0] += a;
        h_[1] += bb;
        h_[2] += c;
        h_[3] += d;
        h_[4] += e;
        h_[5] += f;
        h_[6] += g;
        h_[7] += h;
    }

    uint32_t h_[8];
    uint64_t length_;
    uint8_t block_[64];
    size_t fill_;
};

}  // namespace decisive
