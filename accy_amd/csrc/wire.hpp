// ACTP v1 wire bytes: the language-neutral encoding of a tensor program.
// Layout restated from src/tensor/wire/format.zig:1-113, encode.zig:28-230, decode.zig:31-120.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "ir.hpp"

namespace accy::wire {

constexpr uint32_t kMagic = 0x50544341u;  // "ACTP" read as a little-endian u32 (format.zig:20)
constexpr uint32_t kVersion = 1;           // format.zig:23
constexpr size_t kMaxScanDepth = 8;        // format.zig:27

// Rebuilds a program from wire bytes, deriving every result type through Builder. Throws accy::Error
// with BadMagic, UnsupportedVersion, UnknownTag, InvalidReference, TooManyOperands, ScanTooDeep,
// InvalidArtifact (truncated or trailing bytes) or any builder check failure.
Program decode(const uint8_t* bytes, size_t len);

// Writes a program as version-1 bytes. Throws InvalidProgram when ids are not dense or parameters
// are out of order (encode.zig:149-166), ScanTooDeep past eight nested scans.
std::vector<uint8_t> encode(const Program& program);

}  // namespace accy::wire
