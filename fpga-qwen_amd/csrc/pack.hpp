// QWCPU01 weight pack: read-only mapping with the reference validator's checks,
// and a seeded random-init writer for synthetic workloads.
//
// Format (engine/INTERFACE.md:8-21): `weights.bin` starts with ASCII "QWCPU01"
// plus 57 zero bytes; tensors are little-endian, 64-byte aligned and disjoint.
// `weights.bin.index` is "QWCPU01 310" then 310 rows
// `name dtype rows cols offset length`; 2D matrices are F16, 1D norms F32
// with cols = 1. The embedding is stored once and reused as the tied head.
#pragma once
#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace qwen_hip {

struct PackTensor {
    int rows = 0, cols = 0;
    const uint16_t* half = nullptr;  // F16 matrix (cols != 1)
    const float* norm = nullptr;     // F32 vector (cols == 1)
};

// Mapped pack. The constructor maps the file (engine/core.cpp:108-117);
// validate() runs the header/index checks of engine/core.cpp:238-276 with the
// same messages and order. Callers check option ranges in between, as the
// reference does (engine/core.cpp:235-237).
class Pack {
public:
    explicit Pack(const std::string& path);
    void validate();
    ~Pack();
    Pack(const Pack&) = delete;
    Pack& operator=(const Pack&) = delete;
    const PackTensor& tensor(const std::string& name) const;
    const PackTensor& layer(int layer, const char* suffix) const;

private:
    std::string path_;
    void* data_ = nullptr;
    size_t length_ = 0;
    std::map<std::string, PackTensor> tensors_;
};

// Canonical tensor order of the exporter (tools/export_native_cpu_weights.py:29-39):
// embedding, final norm, then per layer the eleven layer tensors.
struct PackEntry { std::string name; int rows, cols; };
std::vector<PackEntry> pack_layout();

// Writes weights.bin, .index and .manifest.json. Matrices are N(0, stddev)
// rounded to FP16 (round-to-nearest-even), norm gains are 1.0f.
// Element e of tensor t draws a Box-Muller pair from the splitmix64 stream
// s_t = mix64(seed + (t+1) * 0xD1B54A32D192ED03): u1 from output 2p+1 and
// u2 from output 2p+2 of that stream, p = e/2; even e takes r*cos, odd r*sin.
// Counter-based, so the file is identical for any thread count.
void write_random_pack(const std::string& path, uint64_t seed, double stddev, int threads);

}  // namespace qwen_hip
