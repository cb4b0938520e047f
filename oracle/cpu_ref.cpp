// ORACLE (test infrastructure only): CPU restatement of engine/core.cpp.
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
// Build: oracle/Makefile (g++ -O2 -mavx2 -mfma -mf16c -ffp-contract=off).
#include "cpu_ref.h"

#include <immintrin.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <fcntl.h>
#include <fstream>
#include <functional>
#include <limits>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <sys/mman.h>
#include <sys/stat.h>
#include <thread>
#include <unistd.h>
#include <vector>

namespace {
constexpr int H = 1024, D = 128, Q = 16, K = 8, F = 3072, L = 28, V = 151936;
constexpr size_t kChunk = 512;
void require(bool ok, const std::string& m) {
    if (!ok) throw std::runtime_error(m);
}

// ---- FP16 helpers (F16C: exact widening, round-to-nearest-even narrowing) ----
inline float h2f(uint16_t h) { return _cvtsh_ss(h); }
inline uint16_t f2h(float f) { return _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }

// ---- dot: engine/core.cpp:119-127 ----
// Eight FP32 lanes (lane c accumulates j%8 == c) via fused multiply-add in
// ascending j, then ((c0+c4)+(c1+c5)) + ((c2+c6)+(c3+c7)), which is
// vaddvq_f32(vaddq_f32(a, b)) with a = lanes 0-3 and b = lanes 4-7.
inline float reduce_chains(__m256 acc) {
    const __m128 p = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    alignas(16) float v[4];
    _mm_store_ps(v, p);
    return (v[0] + v[1]) + (v[2] + v[3]);
}
inline __m256 load_half8(const uint16_t* w) {
    return _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(w)));
}
float dot(const float* x, const uint16_t* w, int n) {
    __m256 acc = _mm256_setzero_ps();
    for (int j = 0; j < n; j += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(x + j), load_half8(w + j), acc);
    return reduce_chains(acc);
}
// NR weight rows x NB activation rows of independent dot() chains sharing
// loads (the role of dot4, engine/core.cpp:131-147); per-output arithmetic is
// exactly dot().
template <int NR, int NB>
void dot_tile(const float* x, size_t xs, const uint16_t* w, size_t ws, int n, float* y, size_t ys) {
    __m256 acc[NR][NB];
    for (int r = 0; r < NR; ++r)
        for (int b = 0; b < NB; ++b) acc[r][b] = _mm256_setzero_ps();
    for (int j = 0; j < n; j += 8) {
        __m256 xv[NB];
        for (int b = 0; b < NB; ++b) xv[b] = _mm256_loadu_ps(x + b * xs + j);
        for (int r = 0; r < NR; ++r) {
            const __m256 wv = load_half8(w + r * ws + j);
            for (int b = 0; b < NB; ++b) acc[r][b] = _mm256_fmadd_ps(xv[b], wv, acc[r][b]);
        }
    }
    for (int r = 0; r < NR; ++r)
        for (int b = 0; b < NB; ++b) y[b * ys + r] = reduce_chains(acc[r][b]);
}
// y[b*rows + r] = dot(x + b*n, w + r*n) for rows [r0, r1) and all batch rows.
void project_rows(const float* x, int batch, const uint16_t* w, int rows, int n, float* y, size_t r0, size_t r1) {
    size_t r = r0;
    for (; r + 4 <= r1; r += 4) {
        int b = 0;
        for (; b + 2 <= batch; b += 2)
            dot_tile<4, 2>(x + size_t(b) * n, n, w + r * n, n, n, y + size_t(b) * rows + r, rows);
        for (; b < batch; ++b) dot_tile<4, 1>(x + size_t(b) * n, n, w + r * n, n, n, y + size_t(b) * rows + r, rows);
    }
    for (; r < r1; ++r)
        for (int b = 0; b < batch; ++b) y[size_t(b) * rows + r] = dot(x + size_t(b) * n, w + r * n, n);
}

// ---- norm: engine/core.cpp:207-215 ----
void norm(const float* x, const float* w, float* out, int n) {
    double precise_sum = 0;
    for (int j = 0; j < n; ++j) {
        const float square = x[j] * x[j];
        precise_sum += static_cast<double>(square);
    }
    const float sum = static_cast<float>(precise_sum);
    const float inv = 1.0f / std::sqrt(sum / n + 1e-6f);
    for (int j = 0; j < n; ++j) out[j] = (x[j] * inv) * w[j];
}

// ---- rope: engine/core.cpp:216-218 (evaluated as written, no contraction) ----
void rope(float* x, const float* cs, const float* sn) {
    for (int j = 0; j < 64; ++j) {
        const float a = x[j], b = x[j + 64];
        x[j] = a * cs[j] - b * sn[j];
        x[j + 64] = b * cs[j] + a * sn[j];
    }
}
// Tables: engine/core.cpp:287-288 (angle in double, stored as FP32).
void rope_tables(int context, float* cs, float* sn) {
    for (int p = 0; p < context; ++p)
        for (int j = 0; j < 64; ++j) {
            const double angle = p / std::pow(1000000.0, 2.0 * j / D);
            cs[p * 64 + j] = float(std::cos(angle));
            sn[p * 64 + j] = float(std::sin(angle));
        }
}

// ---- decode attention for one head: engine/core.cpp:610-622 ----
// keys/values: rows of 128 FP16 at the given stride (in elements).
void attend(const float* query, const uint16_t* keys, const uint16_t* values, size_t stride, int n, float* scores,
            float* probs, float* dest) {
    const float scale = 1.0f / std::sqrt(float(D));
    float maximum = -std::numeric_limits<float>::infinity();
    for (int t = 0; t < n; ++t) {
        const float s = dot(query, keys + t * stride, D) * scale;
        scores[t] = s;
        maximum = std::max(maximum, s);
    }
    for (int t = 0; t < n; ++t) probs[t] = std::exp(scores[t] - maximum);  // vvexpf -> glibc expf
    float sum = 0;
    for (int t = 0; t < n; ++t) sum += probs[t];
    __m256 acc[16];
    for (int c = 0; c < 16; ++c) acc[c] = _mm256_setzero_ps();
    for (int t = 0; t < n; ++t) {
        const float prob = probs[t] / sum;
        const __m256 p = _mm256_set1_ps(prob);
        const uint16_t* val = values + t * stride;
        for (int c = 0; c < 16; ++c) acc[c] = _mm256_fmadd_ps(load_half8(val + 8 * c), p, acc[c]);
    }
    for (int c = 0; c < 16; ++c) _mm256_storeu_ps(dest + 8 * c, acc[c]);
}

// ---- SwiGLU: engine/core.cpp:636-639 (vvtanhf -> glibc tanhf) ----
void swiglu(const float* gate, const float* up, float* out, int n) {
    for (int j = 0; j < n; ++j) {
        const float half_gate = gate[j] * 0.5f;
        const float t = std::tanh(half_gate);
        out[j] = gate[j] * (0.5f + 0.5f * t) * up[j];
    }
}

// ---- persistent worker pool: rows split as count*i/n (engine/core.cpp:68,96) ----
class Pool {
public:
    explicit Pool(int n) : n_(n) {
        for (int i = 1; i < n_; ++i) threads_.emplace_back([this, i] { work(i); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> lock(mutex_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto& t : threads_) t.join();
    }
    void run(size_t count, const std::function<void(size_t, size_t)>& fn) {
        {
            std::lock_guard<std::mutex> lock(mutex_);
            job_ = &fn;
            count_ = count;
            done_.store(0, std::memory_order_relaxed);
            generation_.fetch_add(1, std::memory_order_release);
        }
        cv_.notify_all();
        fn(0, count / n_);
        while (done_.load(std::memory_order_acquire) != n_ - 1) _mm_pause();
        job_ = nullptr;
    }

private:
    void work(int i) {
        uint64_t seen = 0;
        for (;;) {
            const auto deadline = std::chrono::steady_clock::now() + std::chrono::microseconds(50);
            while (generation_.load(std::memory_order_acquire) == seen && !stop_) {
                _mm_pause();
                if (std::chrono::steady_clock::now() >= deadline) break;
            }
            {
                std::unique_lock<std::mutex> lock(mutex_);
                cv_.wait(lock, [&] { return stop_ || generation_.load(std::memory_order_acquire) != seen; });
                if (stop_) return;
            }
            seen = generation_.load(std::memory_order_acquire);
            const size_t count = count_;
            (*job_)(count * i / n_, count * (i + 1) / n_);
            done_.fetch_add(1, std::memory_order_acq_rel);
        }
    }
    int n_;
    std::vector<std::thread> threads_;
    std::mutex mutex_;
    std::condition_variable cv_;
    std::atomic<uint64_t> generation_{0};
    std::atomic<int> done_{0};
    const std::function<void(size_t, size_t)>* job_ = nullptr;
    size_t count_ = 0;
    bool stop_ = false;
};

struct Layer {
    const float *in_norm, *post_norm, *q_norm, *k_norm;
    const uint16_t *q, *k, *v, *o, *gate, *up, *down;
};

}  // namespace

struct cpuref_model {
    int decode_threads, prefill_threads, context;
    void* map = nullptr;
    size_t map_len = 0;
    const uint16_t* embed = nullptr;
    const float* final_norm = nullptr;
    std::array<Layer, L> layers{};
    std::vector<uint16_t> keys, values;  // [layer][kv head][position][128]
    std::vector<float> cosines, sines;
    std::unique_ptr<Pool> decode_pool, prefill_pool;
    std::vector<float> x, h, q, k, v, attended, residual, gate, up, act;
    std::vector<float> scores, probs;  // per worker [context]
    std::array<float, H> last_hidden{};
    std::vector<float> output;
    int pos = 0;
    std::string error;

    size_t cache_offset(int layer, int position, int head) const {
        return ((size_t(layer) * K + head) * context + position) * D;
    }

    cpuref_model(const std::string& path, int dt, int pt, int ctx)
        : decode_threads(dt), prefill_threads(pt), context(ctx) {
        require(dt >= 1 && dt <= 64 && pt >= 1 && pt <= 64, "Threads must be in 1..64");
        require(ctx >= 1 && ctx <= 4096, "Context must be in 1..4096");
        const int fd = ::open(path.c_str(), O_RDONLY);
        require(fd >= 0, "Cannot open weights");
        struct stat st {};
        require(::fstat(fd, &st) == 0 && st.st_size >= 64, "Invalid weights size");
        map_len = size_t(st.st_size);
        map = ::mmap(nullptr, map_len, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        require(map != MAP_FAILED, "Cannot mmap weights");
        require(std::memcmp(map, "QWCPU01", 7) == 0, "Invalid weight pack header");
        std::ifstream index(path + ".index");
        std::string sig;
        size_t count = 0;
        require(bool(index >> sig >> count) && sig == "QWCPU01" && count == 310, "Invalid weight index header/count");
        std::map<std::string, const unsigned char*> ptr;
        std::map<std::string, std::pair<uint64_t, uint64_t>> shape;
        for (size_t i = 0; i < count; ++i) {
            std::string name, type;
            uint64_t rows, cols, offset, length;
            require(bool(index >> name >> type >> rows >> cols >> offset >> length), "Truncated weight index");
            require(offset + length <= map_len, "Invalid tensor range: " + name);
            ptr[name] = static_cast<const unsigned char*>(map) + offset;
            shape[name] = {rows, cols};
        }
        auto mat = [&](const std::string& n, uint64_t r, uint64_t c) {
            require(ptr.count(n) && shape[n] == std::make_pair(r, c), "Wrong tensor shape: " + n);
            return reinterpret_cast<const uint16_t*>(ptr[n]);
        };
        auto vec = [&](const std::string& n, uint64_t r) {
            require(ptr.count(n) && shape[n] == std::make_pair(r, uint64_t(1)), "Wrong tensor shape: " + n);
            return reinterpret_cast<const float*>(ptr[n]);
        };
        embed = mat("model.embed_tokens.weight", V, H);
        final_norm = vec("model.norm.weight", H);
        for (int l = 0; l < L; ++l) {
            const std::string p = "model.layers." + std::to_string(l) + ".";
            Layer& y = layers[l];
            y.in_norm = vec(p + "input_layernorm.weight", H);
            y.post_norm = vec(p + "post_attention_layernorm.weight", H);
            y.q_norm = vec(p + "self_attn.q_norm.weight", D);
            y.k_norm = vec(p + "self_attn.k_norm.weight", D);
            y.q = mat(p + "self_attn.q_proj.weight", Q * D, H);
            y.k = mat(p + "self_attn.k_proj.weight", K * D, H);
            y.v = mat(p + "self_attn.v_proj.weight", K * D, H);
            y.o = mat(p + "self_attn.o_proj.weight", H, Q * D);
            y.gate = mat(p + "mlp.gate_proj.weight", F, H);
            y.up = mat(p + "mlp.up_proj.weight", F, H);
            y.down = mat(p + "mlp.down_proj.weight", H, F);
        }
        keys.resize(size_t(L) * ctx * K * D);
        values.resize(keys.size());
        cosines.resize(size_t(ctx) * 64);
        sines.resize(cosines.size());
        rope_tables(ctx, cosines.data(), sines.data());
        const int workers = std::max(dt, pt);
        scores.resize(size_t(workers) * ctx);
        probs.resize(scores.size());
        decode_pool = std::make_unique<Pool>(dt);
        prefill_pool = std::make_unique<Pool>(pt);
    }
    ~cpuref_model() {
        decode_pool.reset();
        prefill_pool.reset();
        if (map && map != MAP_FAILED) ::munmap(map, map_len);
    }

    void project(const uint16_t* w, int rows, int n, const float* in, float* out, int batch, Pool& pool) {
        pool.run(size_t(rows), [&](size_t b, size_t e) { project_rows(in, batch, w, rows, n, out, b, e); });
    }

    // engine/core.cpp:353-646, with per-row B1 arithmetic for every projection.
    void chunk(const int* ids, int batch, Pool& pool) {
        x.resize(size_t(batch) * H);
        h.resize(x.size());
        q.resize(size_t(batch) * Q * D);
        k.resize(size_t(batch) * K * D);
        v.resize(k.size());
        attended.resize(q.size());
        residual.resize(x.size());
        gate.resize(size_t(batch) * F);
        up.resize(gate.size());
        act.resize(gate.size());
        for (int b = 0; b < batch; ++b)
            for (int j = 0; j < H; ++j) x[size_t(b) * H + j] = h2f(embed[size_t(ids[b]) * H + j]);
        for (int layer = 0; layer < L; ++layer) {
            const Layer& w = layers[layer];
            for (int b = 0; b < batch; ++b) norm(x.data() + size_t(b) * H, w.in_norm, h.data() + size_t(b) * H, H);
            project(w.q, Q * D, H, h.data(), q.data(), batch, pool);
            project(w.k, K * D, H, h.data(), k.data(), batch, pool);
            project(w.v, K * D, H, h.data(), v.data(), batch, pool);
            for (int b = 0; b < batch; ++b) {
                const float* cs = cosines.data() + size_t(pos + b) * 64;
                const float* sn = sines.data() + size_t(pos + b) * 64;
                for (int head = 0; head < Q; ++head) {
                    float* a = q.data() + (size_t(b) * Q + head) * D;
                    norm(a, w.q_norm, a, D);
                    rope(a, cs, sn);
                }
                for (int head = 0; head < K; ++head) {
                    float* a = k.data() + (size_t(b) * K + head) * D;
                    norm(a, w.k_norm, a, D);
                    rope(a, cs, sn);
                }
                for (int head = 0; head < K; ++head) {
                    const size_t dst = cache_offset(layer, pos + b, head), src = (size_t(b) * K + head) * D;
                    for (int j = 0; j < D; ++j) {
                        keys[dst + j] = f2h(k[src + j]);
                        values[dst + j] = f2h(v[src + j]);
                    }
                }
            }
            // Items are (row, head); worker w owns its contiguous item slice.
            std::atomic<int> slot{0};
            pool.run(size_t(batch) * Q, [&](size_t begin, size_t end) {
                const int s = slot.fetch_add(1);
                float* sc = scores.data() + size_t(s) * context;
                float* pr = probs.data() + size_t(s) * context;
                for (size_t item = begin; item < end; ++item) {
                    const int b = int(item / Q), head = int(item % Q), kh = head / 2, n = pos + b + 1;
                    attend(q.data() + item * D, keys.data() + cache_offset(layer, 0, kh),
                           values.data() + cache_offset(layer, 0, kh), D, n, sc, pr, attended.data() + item * D);
                }
            });
            project(w.o, H, Q * D, attended.data(), residual.data(), batch, pool);
            for (size_t j = 0; j < x.size(); ++j) x[j] += residual[j];
            for (int b = 0; b < batch; ++b) norm(x.data() + size_t(b) * H, w.post_norm, h.data() + size_t(b) * H, H);
            project(w.gate, F, H, h.data(), gate.data(), batch, pool);
            project(w.up, F, H, h.data(), up.data(), batch, pool);
            swiglu(gate.data(), up.data(), act.data(), batch * F);
            project(w.down, H, F, act.data(), residual.data(), batch, pool);
            for (size_t j = 0; j < x.size(); ++j) x[j] += residual[j];
        }
        pos += batch;
        norm(x.data() + size_t(batch - 1) * H, final_norm, last_hidden.data(), H);
    }

    // engine/core.cpp:707-714
    void append(const int* ids, size_t count, bool prefill) {
        require(count > 0, "Empty token input");
        require(count <= size_t(context - pos), "Context capacity exceeded");
        for (size_t i = 0; i < count; ++i) require(ids[i] >= 0 && ids[i] < V, "Token ID out of range");
        Pool& pool = prefill ? *prefill_pool : *decode_pool;
        for (size_t begin = 0; begin < count; begin += kChunk)
            chunk(ids + begin, int(std::min(kChunk, count - begin)), pool);
        output.resize(V);
        project(embed, V, H, last_hidden.data(), output.data(), 1, pool);
    }
};

extern "C" {

cpuref_model* cpuref_create(const char* weights, int dt, int pt, int ctx, char* error, size_t error_len) {
    try {
        return new cpuref_model(weights, dt, pt, ctx);
    } catch (const std::exception& e) {
        if (error && error_len) {
            std::strncpy(error, e.what(), error_len - 1);
            error[error_len - 1] = 0;
        }
        return nullptr;
    }
}
void cpuref_destroy(cpuref_model* m) { delete m; }
const char* cpuref_error(const cpuref_model* m) { return m->error.c_str(); }

#define CPUREF_GUARD(body)                 \
    try {                                  \
        body;                              \
        return 0;                          \
    } catch (const std::exception& e) {    \
        m->error = e.what();               \
        return 1;                          \
    }

int cpuref_reset(cpuref_model* m) { CPUREF_GUARD({ m->pos = 0; m->output.clear(); }) }
int cpuref_truncate(cpuref_model* m, int position) {
    CPUREF_GUARD({
        require(position >= 0 && position <= m->pos, "Rewind position out of range");
        m->pos = position;
        m->output.clear();
    })
}
int cpuref_prefill(cpuref_model* m, const int* ids, size_t count) { CPUREF_GUARD(m->append(ids, count, true)) }
int cpuref_step(cpuref_model* m, int token) { CPUREF_GUARD(m->append(&token, 1, false)) }
int cpuref_position(const cpuref_model* m) { return m->pos; }
const float* cpuref_logits(const cpuref_model* m) { return m->output.size() == size_t(V) ? m->output.data() : nullptr; }
const float* cpuref_hidden(const cpuref_model* m) {
    return (m->pos > 0 && m->output.size() == size_t(V)) ? m->last_hidden.data() : nullptr;
}

float cpuref_dot(const float* x, const uint16_t* w, int n) { return dot(x, w, n); }
void cpuref_gemv(const float* x, const uint16_t* w, float* y, int rows, int n, int threads) {
    Pool pool(std::max(1, threads));
    pool.run(size_t(rows), [&](size_t b, size_t e) { project_rows(x, 1, w, rows, n, y, b, e); });
}
void cpuref_norm(const float* x, const float* w, float* out, int n) { norm(x, w, out, n); }
void cpuref_rope_tables(int context, float* cs, float* sn) { rope_tables(context, cs, sn); }
void cpuref_rope(float* x, const float* cs, const float* sn) { rope(x, cs, sn); }
void cpuref_attention(const float* q, const uint16_t* keys, const uint16_t* values, int n, float* out) {
    std::vector<float> s(size_t(std::max(n, 1))), p(s.size());
    attend(q, keys, values, D, n, s.data(), p.data(), out);
}
void cpuref_swiglu(const float* gate, const float* up, float* out, int n) { swiglu(gate, up, out, n); }
int cpuref_argmax(const float* logits, int n) {
    int best = 0;
    for (int id = 0; id < n; ++id) {
        if (!std::isfinite(logits[id])) return -1;
        if (logits[id] > logits[best]) best = id;
    }
    return best;
}
uint16_t cpuref_f32_to_f16(float x) { return f2h(x); }
float cpuref_f16_to_f32(uint16_t h) { return h2f(h); }

}  // extern "C"
