// QWCPU01 pack mapping/validation and the seeded random-init pack writer.
#include "pack.hpp"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <fcntl.h>
#include <fstream>
#include <sys/mman.h>
#include <sys/stat.h>
#include <thread>
#include <unistd.h>

#include "qwen_common.hpp"

namespace qwen_hip {
namespace {

// IEEE binary32 -> binary16, round to nearest even; overflow becomes infinity.
uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return uint16_t(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return uint16_t(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        // Below the smallest normal half: scale by 2^24 (exact) and round.
        const float scaled = std::fabs(f) * 16777216.0f;
        return uint16_t(sign | uint32_t(std::nearbyint(scaled)));
    }
    ax -= 0x38000000u;  // rebias exponent 127 -> 15
    return uint16_t(sign | ((ax + 0x0fffu + ((ax >> 13) & 1u)) >> 13));
}

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

}  // namespace

std::vector<PackEntry> pack_layout() {
    std::vector<PackEntry> out;
    out.push_back({"model.embed_tokens.weight", kVocab, kHidden});
    out.push_back({"model.norm.weight", kHidden, 1});
    for (int l = 0; l < kLayers; ++l) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        out.push_back({p + "input_layernorm.weight", kHidden, 1});
        out.push_back({p + "post_attention_layernorm.weight", kHidden, 1});
        out.push_back({p + "self_attn.q_norm.weight", kHeadDim, 1});
        out.push_back({p + "self_attn.k_norm.weight", kHeadDim, 1});
        out.push_back({p + "self_attn.q_proj.weight", kQDim, kHidden});
        out.push_back({p + "self_attn.k_proj.weight", kKVDim, kHidden});
        out.push_back({p + "self_attn.v_proj.weight", kKVDim, kHidden});
        out.push_back({p + "self_attn.o_proj.weight", kHidden, kQDim});
        out.push_back({p + "mlp.gate_proj.weight", kFFN, kHidden});
        out.push_back({p + "mlp.up_proj.weight", kFFN, kHidden});
        out.push_back({p + "mlp.down_proj.weight", kHidden, kFFN});
    }
    return out;
}

Pack::Pack(const std::string& path) : path_(path) {
    // Mapping errors (engine/core.cpp:110-114).
    const int fd = ::open(path.c_str(), O_RDONLY);
    require(fd >= 0, "Cannot open weights");
    struct stat st {};
    if (::fstat(fd, &st) != 0 || st.st_size < 64) {
        ::close(fd);
        throw std::runtime_error("Invalid weights size");
    }
    length_ = size_t(st.st_size);
    data_ = ::mmap(nullptr, length_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (data_ == MAP_FAILED) {
        data_ = nullptr;
        throw std::runtime_error("Cannot mmap weights");
    }
}

void Pack::validate() {
    const std::string& path = path_;
    try {
        // Header and index validation (engine/core.cpp:238-276), same order.
        std::array<unsigned char, 64> magic{};
        std::memcpy(magic.data(), "QWCPU01", 7);
        require(std::memcmp(data_, magic.data(), 64) == 0, "Invalid weight pack header");
        std::map<std::string, std::pair<int, int>> expected;
        for (const auto& e : pack_layout()) expected[e.name] = {e.rows, e.cols};
        std::ifstream index(path + ".index");
        std::string signature;
        size_t count = 0;
        require(bool(index >> signature >> count) && signature == "QWCPU01" && count == expected.size(),
                "Invalid weight index header/count");
        std::vector<std::pair<size_t, size_t>> ranges;
        const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
        for (size_t i = 0; i < count; ++i) {
            std::string name, type;
            uint64_t rows, cols, offset, length;
            require(bool(index >> name >> type >> rows >> cols >> offset >> length), "Truncated weight index");
            auto it = expected.find(name);
            require(it != expected.end() && !tensors_.count(name), "Unexpected or duplicate tensor: " + name);
            require(rows == uint64_t(it->second.first) && cols == uint64_t(it->second.second),
                    "Wrong tensor shape: " + name);
            const bool matrix = cols != 1;
            require(type == (matrix ? "F16" : "F32"), "Wrong tensor dtype: " + name);
            require(length == rows * cols * (matrix ? 2 : 4) && offset >= 64 && offset % 64 == 0 &&
                        offset <= length_ && length <= length_ - offset,
                    "Invalid tensor range: " + name);
            ranges.emplace_back(offset, offset + length);
            PackTensor t;
            t.rows = int(rows);
            t.cols = int(cols);
            const auto* bytes = static_cast<const unsigned char*>(data_) + offset;
            if (matrix) {
                t.half = reinterpret_cast<const uint16_t*>(bytes);
                // Finite FP16 <=> exponent field not all ones.
                const size_t n = size_t(rows) * cols;
                const unsigned workers = n > (1u << 22) ? hw : 1u;
                std::vector<char> bad(workers, 0);
                std::vector<std::thread> pool;
                for (unsigned w = 0; w < workers; ++w)
                    pool.emplace_back([&, w] {
                        const size_t b = n * w / workers, e = n * (w + 1) / workers;
                        for (size_t j = b; j < e; ++j)
                            if ((t.half[j] & 0x7c00u) == 0x7c00u) { bad[w] = 1; break; }
                    });
                for (auto& th : pool) th.join();
                require(std::find(bad.begin(), bad.end(), 1) == bad.end(), "Nonfinite matrix: " + name);
            } else {
                t.norm = reinterpret_cast<const float*>(bytes);
                for (size_t j = 0; j < rows; ++j) require(std::isfinite(t.norm[j]), "Nonfinite norm: " + name);
            }
            tensors_.emplace(name, t);
        }
        std::string extra;
        require(!(index >> extra), "Trailing weight index data");
        std::sort(ranges.begin(), ranges.end());
        for (size_t i = 1; i < ranges.size(); ++i)
            require(ranges[i].first >= ranges[i - 1].second, "Overlapping tensors");
    } catch (...) {
        ::munmap(data_, length_);
        data_ = nullptr;
        throw;
    }
}

Pack::~Pack() {
    if (data_) ::munmap(data_, length_);
}

const PackTensor& Pack::tensor(const std::string& name) const { return tensors_.at(name); }

const PackTensor& Pack::layer(int layer, const char* suffix) const {
    return tensors_.at("model.layers." + std::to_string(layer) + "." + suffix);
}

void write_random_pack(const std::string& path, uint64_t seed, double stddev, int threads) {
    const auto layout = pack_layout();
    const std::string index_path = path + ".index", manifest_path = path + ".manifest.json";
    for (const auto& p : {path, index_path, manifest_path}) {
        struct stat st {};
        require(::lstat(p.c_str(), &st) != 0, "Weight pack outputs are immutable; choose a fresh path");
    }
    std::vector<size_t> offsets;
    size_t cursor = 64;
    for (const auto& e : layout) {
        cursor = (cursor + 63) / 64 * 64;
        offsets.push_back(cursor);
        cursor += size_t(e.rows) * e.cols * (e.cols == 1 ? 4 : 2);
    }
    const size_t total = cursor;
    const int fd = ::open(path.c_str(), O_RDWR | O_CREAT | O_EXCL, 0644);
    require(fd >= 0, "Cannot create weight pack");
    if (::ftruncate(fd, off_t(total)) != 0) {
        ::close(fd);
        throw std::runtime_error("Cannot size weight pack");
    }
    void* map = ::mmap(nullptr, total, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
    ::close(fd);
    require(map != MAP_FAILED, "Cannot map weight pack for writing");
    auto* base = static_cast<unsigned char*>(map);
    std::memset(base, 0, 64);
    std::memcpy(base, "QWCPU01", 7);
    const int workers = std::max(1, std::min(threads, 64));
    std::vector<std::thread> pool;
    for (int w = 0; w < workers; ++w) {
        pool.emplace_back([&, w] {
            for (size_t t = 0; t < layout.size(); ++t) {
                const auto& e = layout[t];
                const size_t n = size_t(e.rows) * e.cols;
                const size_t b = n * w / workers, end = n * (w + 1) / workers;
                if (e.cols == 1) {
                    float* dst = reinterpret_cast<float*>(base + offsets[t]);
                    for (size_t j = b; j < end; ++j) dst[j] = 1.0f;
                    continue;
                }
                uint16_t* dst = reinterpret_cast<uint16_t*>(base + offsets[t]);
                const uint64_t stream = mix64(seed + (uint64_t(t) + 1) * 0xD1B54A32D192ED03ull);
                // Pairs [2p, 2p+1] share one Box-Muller draw; slice ends may split a pair.
                for (size_t j = b; j < end;) {
                    const uint64_t pair = j >> 1;
                    const uint64_t a = mix64(stream + (2 * pair + 1) * kGolden);
                    const uint64_t c = mix64(stream + (2 * pair + 2) * kGolden);
                    const double u1 = double((a >> 11) + 1) * 0x1.0p-53;  // (0, 1]
                    const double u2 = double(c >> 11) * 0x1.0p-53;        // [0, 1)
                    const double r = std::sqrt(-2.0 * std::log(u1));
                    const double theta = 6.283185307179586476925286766559 * u2;
                    if (!(j & 1)) {
                        dst[j] = f32_to_f16(float(stddev * (r * std::cos(theta))));
                        if (++j >= end) break;
                    }
                    dst[j] = f32_to_f16(float(stddev * (r * std::sin(theta))));
                    ++j;
                }
            }
        });
    }
    for (auto& th : pool) th.join();
    ::msync(map, total, MS_SYNC);
    ::munmap(map, total);
    {
        std::ofstream index(index_path);
        index << "QWCPU01 " << layout.size() << "\n";
        for (size_t t = 0; t < layout.size(); ++t) {
            const auto& e = layout[t];
            const size_t bytes = size_t(e.rows) * e.cols * (e.cols == 1 ? 4 : 2);
            index << e.name << ' ' << (e.cols == 1 ? "F32" : "F16") << ' ' << e.rows << ' ' << e.cols << ' '
                  << offsets[t] << ' ' << bytes << "\n";
        }
        require(bool(index), "Failed writing weight index");
    }
    {
        std::ofstream manifest(manifest_path);
        manifest << "{\n  \"format\": \"QWCPU01\",\n  \"completed\": true,\n  \"tensor_count\": " << layout.size()
                 << ",\n  \"binary\": {\"path\": \"" << path.substr(path.find_last_of('/') + 1)
                 << "\", \"bytes\": " << total << "},\n  \"synthetic\": {\"generator\": \"splitmix64-box-muller\", "
                 << "\"seed\": " << seed << ", \"stddev\": " << stddev << ", \"norm_gain\": 1.0},\n"
                 << "  \"tied_lm_head_verified\": true,\n"
                 << "  \"rounding\": \"N(0, stddev) in FP64, rounded to FP32, then FP16 round-to-nearest-even; "
                    "1D norms FP32 1.0; little endian\"\n}\n";
        require(bool(manifest), "Failed writing weight manifest");
    }
}

}  // namespace qwen_hip
