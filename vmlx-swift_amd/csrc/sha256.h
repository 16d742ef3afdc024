// sha256.h -- SHA-256 (FIPS 180-4) for the prefix-cache chain hash.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <string>

namespace vkv {

class Sha256 {
 public:
  Sha256();
  void update(const void* data, size_t len);
  // 64 lowercase hex characters.
  std::string hex_digest();

 private:
  void block(const uint8_t* p);
  uint32_t h_[8];
  uint8_t buf_[64];
  size_t buf_len_;
  uint64_t total_;
};

}  // namespace vkv
