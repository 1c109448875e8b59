// aos_determinism.hpp — the seeds and hashes the router's determinism features are built from,
// restated for the C++ host side:
//   B3Hash                    crates/adapteros-infra-common/src/hash.rs (BLAKE3 via aoship_blake3;
//                             from_hex / to_hex / to_short_hex)
//   derive_seed               crates/adapteros-core/src/seed.rs:986-1006 (HKDF-SHA256, no salt,
//                             IKM = the global seed, info = the label, 32 bytes)
//   derive_router_seed        crates/adapteros-core/src/determinism.rs:138-150 (label "router" or
//                             "router:<manifest hash hex>", hex encoded)
//   derive_router_tiebreak_seed
//                             crates/adapteros-core/src/determinism.rs:172-176 (label "router-tie"
//                             over the router seed, parsed as hex, else BLAKE3 of its text)
//   DeterminismContext        crates/adapteros-core/src/determinism.rs:17-135
// SHA-256 (FIPS 180-4), HMAC (RFC 2104) and HKDF (RFC 5869) are written here from their
// specifications; the reference takes them from the sha2 0.10 / hmac / hkdf 0.12 crates. The
// global fixed_seed override of the determinism config (seed.rs:988-999) is not modelled.
#pragma once

#include <array>
#include <cstdint>
#include <cstring>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/aoship.h"

namespace adapteros {
namespace det {

using Bytes32 = std::array<uint8_t, 32>;

// ---- SHA-256 -------------------------------------------------------------------------------------

class Sha256 {
 public:
  Sha256() { reset(); }
  void reset() {
    static const uint32_t h0[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                                   0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    memcpy(h_, h0, sizeof h_);
    len_ = 0;
    fill_ = 0;
  }
  void update(const uint8_t *p, size_t n) {
    len_ += n;
    while (n) {
      const size_t take = n < 64 - fill_ ? n : 64 - fill_;
      memcpy(buf_ + fill_, p, take);
      fill_ += take;
      p += take;
      n -= take;
      if (fill_ == 64) {
        block(buf_);
        fill_ = 0;
      }
    }
  }
  void update(const std::string &s) { update((const uint8_t *)s.data(), s.size()); }
  Bytes32 digest() {
    const uint64_t bits = len_ * 8;
    const uint8_t one = 0x80, zero = 0;
    update(&one, 1);
    while (fill_ != 56) update(&zero, 1);
    uint8_t lb[8];
    for (int i = 0; i < 8; ++i) lb[i] = (uint8_t)(bits >> (56 - 8 * i));
    update(lb, 8);
    Bytes32 out;
    for (int i = 0; i < 8; ++i)
      for (int b = 0; b < 4; ++b) out[(size_t)(4 * i + b)] = (uint8_t)(h_[i] >> (24 - 8 * b));
    reset();
    return out;
  }

 private:
  static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
  void block(const uint8_t *p) {
    static const uint32_t k[64] = {
        0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
        0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
        0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
        0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
        0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
        0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
        0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
        0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};
    uint32_t w[64];
    for (int i = 0; i < 16; ++i)
      w[i] = ((uint32_t)p[4 * i] << 24) | ((uint32_t)p[4 * i + 1] << 16) | ((uint32_t)p[4 * i + 2] << 8) | p[4 * i + 3];
    for (int i = 16; i < 64; ++i) {
      const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
      const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
      w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h_[0], b = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], h = h_[7];
    for (int i = 0; i < 64; ++i) {
      const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[i] + w[i];
      const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
      h = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = b;
      b = a;
      a = t1 + t2;
    }
    h_[0] += a;
    h_[1] += b;
    h_[2] += c;
    h_[3] += d;
    h_[4] += e;
    h_[5] += f;
    h_[6] += g;
    h_[7] += h;
  }
  uint32_t h_[8];
  uint64_t len_;
  uint8_t buf_[64];
  size_t fill_;
};

inline Bytes32 sha256(const uint8_t *p, size_t n) {
  Sha256 s;
  s.update(p, n);
  return s.digest();
}

// HMAC-SHA256 (RFC 2104): keys longer than the 64-byte block are hashed first.
inline Bytes32 hmac_sha256(const uint8_t *key, size_t klen, const uint8_t *msg, size_t mlen) {
  uint8_t k[64] = {0};
  if (klen > 64) {
    const Bytes32 kh = sha256(key, klen);
    memcpy(k, kh.data(), 32);
  } else if (klen) {
    memcpy(k, key, klen);
  }
  uint8_t ipad[64], opad[64];
  for (int i = 0; i < 64; ++i) {
    ipad[i] = (uint8_t)(k[i] ^ 0x36);
    opad[i] = (uint8_t)(k[i] ^ 0x5c);
  }
  Sha256 in;
  in.update(ipad, 64);
  in.update(msg, mlen);
  const Bytes32 ih = in.digest();
  Sha256 out;
  out.update(opad, 64);
  out.update(ih.data(), 32);
  return out.digest();
}

// HKDF-SHA256 (RFC 5869): extract with salt (empty / absent = 32 zero bytes), expand to len
// bytes (len <= 255 * 32).
inline std::vector<uint8_t> hkdf_sha256(const uint8_t *salt, size_t slen, const uint8_t *ikm, size_t ilen,
                                        const uint8_t *info, size_t nlen, size_t len) {
  if (len > 255 * 32) throw std::invalid_argument("HKDF output too long");
  const uint8_t zero[32] = {0};
  const Bytes32 prk = slen ? hmac_sha256(salt, slen, ikm, ilen) : hmac_sha256(zero, 32, ikm, ilen);
  std::vector<uint8_t> okm, t;
  for (uint8_t i = 1; okm.size() < len; ++i) {
    std::vector<uint8_t> m(t);
    m.insert(m.end(), info, info + nlen);
    m.push_back(i);
    const Bytes32 ti = hmac_sha256(prk.data(), 32, m.data(), m.size());
    t.assign(ti.begin(), ti.end());
    okm.insert(okm.end(), t.begin(), t.end());
  }
  okm.resize(len);
  return okm;
}

// ---- B3Hash ----------------------------------------------------------------------------------------

struct B3Hash {
  Bytes32 bytes{};

  static B3Hash hash(const uint8_t *p, size_t n) {
    B3Hash h;
    if (aoship_blake3(n ? p : (const uint8_t *)"", n, h.bytes.data()) != 0)
      throw std::runtime_error(std::string("aoship_blake3: ") + aoship_get_last_error());
    return h;
  }
  static B3Hash hash(const std::string &s) { return hash((const uint8_t *)s.data(), s.size()); }
  // B3Hash::from_hex: hex::decode (either case) of exactly 32 bytes, else nullopt.
  static std::optional<B3Hash> from_hex(const std::string &s) {
    if (s.size() != 64) return std::nullopt;
    B3Hash h;
    for (size_t i = 0; i < 32; ++i) {
      int v = 0;
      for (int j = 0; j < 2; ++j) {
        const char c = s[2 * i + (size_t)j];
        int d;
        if (c >= '0' && c <= '9') d = c - '0';
        else if (c >= 'a' && c <= 'f') d = c - 'a' + 10;
        else if (c >= 'A' && c <= 'F') d = c - 'A' + 10;
        else return std::nullopt;
        v = v * 16 + d;
      }
      h.bytes[i] = (uint8_t)v;
    }
    return h;
  }
  std::string to_hex() const { return hex(bytes.data(), 32); }
  std::string to_short_hex() const { return hex(bytes.data(), 8); }  // first 8 bytes (hash.rs:57-59)
  static std::string hex(const uint8_t *p, size_t n) {
    static const char *digits = "0123456789abcdef";
    std::string s;
    for (size_t i = 0; i < n; ++i) {
      s += digits[p[i] >> 4];
      s += digits[p[i] & 15];
    }
    return s;
  }
  bool operator==(const B3Hash &o) const { return bytes == o.bytes; }
};

// ---- seeds ------------------------------------------------------------------------------------------

// derive_seed(global, label) (seed.rs:986-1006)
inline Bytes32 derive_seed(const B3Hash &global, const std::string &label) {
  const std::vector<uint8_t> okm =
      hkdf_sha256(nullptr, 0, global.bytes.data(), 32, (const uint8_t *)label.data(), label.size(), 32);
  Bytes32 out;
  memcpy(out.data(), okm.data(), 32);
  return out;
}

// derive_router_seed (determinism.rs:138-150)
inline std::string derive_router_seed(const Bytes32 &request_seed, const B3Hash *manifest_hash) {
  B3Hash global;
  global.bytes = request_seed;
  const std::string label = manifest_hash ? "router:" + manifest_hash->to_hex() : std::string("router");
  const Bytes32 s = derive_seed(global, label);
  return B3Hash::hex(s.data(), 32);
}

// derive_router_tiebreak_seed (determinism.rs:172-176)
inline Bytes32 derive_router_tiebreak_seed(const std::string &router_seed_hex) {
  const std::optional<B3Hash> parsed = B3Hash::from_hex(router_seed_hex);
  const B3Hash rs = parsed ? *parsed : B3Hash::hash(router_seed_hex);
  return derive_seed(rs, "router-tie");
}

enum class RoutingDeterminismMode { Deterministic, Adaptive };

// DeterminismContext (determinism.rs:17-135): the request seed, the router seed derived from it
// (or given), and the routing mode.
class DeterminismContext {
 public:
  DeterminismContext(const Bytes32 &request_seed, const B3Hash *manifest_hash, RoutingDeterminismMode mode)
      : request_seed_(request_seed), router_seed_hex_(derive_router_seed(request_seed, manifest_hash)), mode_(mode) {}
  DeterminismContext(const Bytes32 &request_seed, std::string router_seed_hex, RoutingDeterminismMode mode)
      : request_seed_(request_seed), router_seed_hex_(std::move(router_seed_hex)), mode_(mode) {}

  const Bytes32 &request_seed() const { return request_seed_; }
  uint64_t request_seed_low64() const {
    uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = (v << 8) | request_seed_[(size_t)i];
    return v;
  }
  const std::string &router_seed_hex() const { return router_seed_hex_; }
  RoutingDeterminismMode routing_mode() const { return mode_; }
  Bytes32 router_tiebreak_seed() const { return derive_router_tiebreak_seed(router_seed_hex_); }

 private:
  Bytes32 request_seed_;
  std::string router_seed_hex_;
  RoutingDeterminismMode mode_;
};

}  // namespace det
}  // namespace adapteros
