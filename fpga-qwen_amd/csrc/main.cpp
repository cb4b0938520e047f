// qwen_gpu: persistent process, protocol v1 (engine/INTERFACE.md:40-90).
// Same argv, commands, JSON responses and error/reset contract as the
// reference CLI (engine/main.cpp:81-195); the engine runs on the GPU, so the
// handshake reports "gpu":true. Greedy selection uses the device argmax
// (identical rule: lowest id among maxima, nonfinite is an error); chat mode
// samples on the host from the copied logits (engine/main.cpp:40-70).
#include <algorithm>
#include <charconv>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <random>
#include <sstream>
#include <string>
#include <vector>

#include "qwen_gpu.hpp"

namespace {
using Clock = std::chrono::steady_clock;
constexpr int kV = qwen_gpu::vocabulary;

std::string json_string(const std::string& value) {
    std::ostringstream out;
    out << '"';
    for (unsigned char c : value) {
        if (c == '"' || c == '\\')
            out << '\\' << c;
        else if (c < 32)
            out << "\\u" << std::hex << std::setw(4) << std::setfill('0') << int(c) << std::dec;
        else
            out << c;
    }
    out << '"';
    return out.str();
}

template <class T>
T parse_integer(const std::string& text) {
    T value{};
    const auto r = std::from_chars(text.data(), text.data() + text.size(), value);
    if (text.empty() || r.ec != std::errc{} || r.ptr != text.data() + text.size())
        throw std::runtime_error("Invalid integer: " + text);
    return value;
}

void no_more(std::istringstream& in) {
    std::string extra;
    if (in >> extra) throw std::runtime_error("Unexpected command argument");
}

bool is_eos(int id) { return id == 151643 || id == 151645; }

// Sampler semantics of engine/main.cpp:40-70: greedy = argmax (lowest id on
// ties); chat = presence penalty 1.5, temperature 0.7, top-k 20, top-p 0.8,
// mt19937_64 seeded per request.
// engine/main.cpp:40-70. The seen set (presence penalty) is kept here and
// mirrored into the model's device flags; the scores and their partial sort
// run on the GPU (qwen_gpu_top_scores), and only the 20 candidates come back
// for the top-p draw below, which is the reference's arithmetic.
class Sampler {
public:
    void reset() {
        std::fill(seen_.begin(), seen_.end(), 0);
        clear_ = true;
        fresh_.clear();
    }
    void mode(bool chat, uint64_t seed) {
        chat_ = chat;
        rng_.seed(seed);
    }
    void consumed(int id) {
        if (!seen_.at(size_t(id))) fresh_.push_back(id);
        seen_[size_t(id)] = 1;
    }
    bool greedy() const { return !chat_; }
    int chat_select(qwen_gpu::Model& model) {
        if (clear_ || !fresh_.empty()) {
            model.update_penalized(clear_, fresh_);
            clear_ = false;
            fresh_.clear();
        }
        float value[kTop];
        int id[kTop];
        model.top_scores(1.5f, .7f, kTop, value, id);
        double p[kTop], total = 0;
        for (int i = 0; i < kTop; ++i) total += (p[i] = std::exp(double(value[i]) - value[0]));
        double kept = 0;
        int count = 0;
        do {
            kept += p[count++];
        } while (count < kTop && kept < .8 * total);
        double draw = std::generate_canonical<double, 53>(rng_) * kept;
        for (int i = 0; i < count; ++i)
            if ((draw -= p[i]) < 0) return id[i];
        return id[count - 1];
    }

private:
    static constexpr int kTop = 20;
    std::vector<unsigned char> seen_ = std::vector<unsigned char>(size_t(kV), 0);
    std::vector<int> fresh_;  // seen since the last upload
    bool clear_ = true;       // the device flags predate the last reset
    std::mt19937_64 rng_{0};
    bool chat_ = false;
};

void handshake(const qwen_gpu::Options& o, const qwen_gpu::Model& model) {
    std::cout << "{\"ready\":true,\"protocol\":1,\"position\":" << model.position()
              << ",\"decode_threads\":" << o.decode_threads << ",\"prefill_threads\":" << o.prefill_threads
              << ",\"context\":" << o.context
              << ",\"lossless_bf16_decode_cache_bytes\":" << model.lossless_bf16_cache_bytes()
              << ",\"gpu\":true,\"pytorch\":false,\"weight_precision\":\"f16\",\"norm_precision\":\"f32\","
                 "\"norm_accumulator_precision\":\"f64\",\"activation_precision\":\"f32\",\"kv_precision\":\"f16\","
                 "\"prefix_reuse\":true,\"prefix_reuse_chunk\":"
              << qwen_gpu::prefix_reuse_chunk
              << ",\"suffix_drafting\":false,\"verify_greedy_b2\":true,\"max_verified_draft\":1}\n"
              << std::flush;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        qwen_gpu::Options options;
        std::string weights;
        for (int i = 1; i < argc; ++i) {
            const std::string key = argv[i];
            if (i + 1 == argc) throw std::runtime_error("Missing option value");
            const std::string value = argv[++i];
            if (key == "--weights")
                weights = value;
            else if (key == "--threads")
                options.decode_threads = parse_integer<int>(value);
            else if (key == "--prefill-threads")
                options.prefill_threads = parse_integer<int>(value);
            else if (key == "--context")
                options.context = parse_integer<int>(value);
            else
                throw std::runtime_error("Unknown option: " + key);
        }
        if (weights.empty()) throw std::runtime_error("--weights is required");
        qwen_gpu::Model model(weights, options);
        Sampler sampler;
        std::vector<int> history;
        history.reserve(size_t(options.context));
        handshake(options, model);
        auto select = [&]() { return sampler.greedy() ? model.greedy() : sampler.chat_select(model); };
        std::string line;
        while (std::getline(std::cin, line)) {
            try {
                if (line.size() > 1024 * 1024 || line.find('\0') != std::string::npos)
                    throw std::runtime_error("Invalid command line");
                std::istringstream in(line);
                std::string command;
                in >> command;
                if (command == "quit") {
                    no_more(in);
                    std::cout << "{\"ok\":true}\n" << std::flush;
                    break;
                }
                if (command == "reset") {
                    no_more(in);
                    model.reset();
                    sampler.reset();
                    history.clear();
                    std::cout << "{\"ok\":true,\"position\":0}\n";
                } else if (command == "rewind") {
                    std::string target;
                    if (!(in >> target)) throw std::runtime_error("Rewind position required");
                    no_more(in);
                    const int keep = parse_integer<int>(target);
                    if (history.size() != size_t(model.position()))
                        throw std::runtime_error("Consumed history does not match model position");
                    model.truncate(keep);  // validates before mutating
                    history.resize(size_t(keep));
                    sampler.reset();
                    for (int id : history) sampler.consumed(id);
                    std::cout << "{\"ok\":true,\"position\":" << keep << "}\n";
                } else if (command == "mode") {
                    std::string mode, seed;
                    in >> mode;
                    if (mode == "greedy") {
                        no_more(in);
                        sampler.mode(false, 0);
                    } else if (mode == "chat") {
                        if (!(in >> seed)) throw std::runtime_error("Chat seed required");
                        no_more(in);
                        sampler.mode(true, parse_integer<uint64_t>(seed));
                    } else {
                        throw std::runtime_error("Unknown decoding mode");
                    }
                    std::cout << "{\"ok\":true}\n";
                } else if (command == "verify-greedy") {
                    std::string pending_text, draft_text;
                    if (!(in >> pending_text >> draft_text))
                        throw std::runtime_error("verify-greedy requires pending and draft IDs");
                    no_more(in);
                    const int pending = parse_integer<int>(pending_text), draft = parse_integer<int>(draft_text);
                    if (!sampler.greedy()) throw std::runtime_error("verify-greedy is unavailable in chat mode");
                    if (history.size() != size_t(model.position()))
                        throw std::runtime_error("Consumed history does not match model position");
                    const auto start = Clock::now();
                    const auto [first, bonus] = model.verify_two_greedy(pending, draft);
                    const bool accepted = first == draft;
                    const int committed = accepted && !is_eos(first) ? 2 : 1;
                    const int second = committed == 2 ? bonus : -1;
                    model.commit_verified(committed);
                    history.push_back(pending);
                    sampler.consumed(pending);
                    if (committed == 2) {
                        history.push_back(draft);
                        sampler.consumed(draft);
                    }
                    const bool stopped = is_eos(first) || (committed == 2 && is_eos(second));
                    const double elapsed = std::chrono::duration<double>(Clock::now() - start).count();
                    std::cout << "{\"tokens\":[" << first;
                    if (committed == 2) std::cout << "," << second;
                    std::cout << "],\"accepted\":" << (accepted ? 1 : 0) << ",\"committed_inputs\":" << committed
                              << ",\"position\":" << model.position()
                              << ",\"verified_positions\":2,\"finish_reason\":" << (stopped ? "\"eos\"" : "null")
                              << ",\"seconds\":" << std::setprecision(17) << elapsed << "}\n";
                } else if (command == "prefill" || command == "step") {
                    std::vector<int> ids;
                    std::string token;
                    while (in >> token) ids.push_back(parse_integer<int>(token));
                    if (ids.empty() || (command == "step" && ids.size() != 1))
                        throw std::runtime_error("Invalid token count");
                    for (int id : ids)
                        if (id < 0 || id >= kV) throw std::runtime_error("Token outside vocabulary");
                    if (ids.size() > size_t(options.context - model.position()))
                        throw std::runtime_error("Context capacity exceeded");
                    if (history.size() != size_t(model.position()))
                        throw std::runtime_error("Consumed history does not match model position");
                    const auto start = Clock::now();
                    if (command == "step")
                        model.step(ids[0]);
                    else
                        model.prefill(ids);
                    history.insert(history.end(), ids.begin(), ids.end());
                    for (int id : ids) sampler.consumed(id);
                    const int selected = select();
                    const double elapsed = std::chrono::duration<double>(Clock::now() - start).count();
                    std::cout << "{\"token\":" << selected << ",\"position\":" << model.position()
                              << ",\"seconds\":" << std::setprecision(17) << elapsed << "}\n";
                } else if (command == "dump-hidden") {
                    const auto space = line.find(' ');
                    if (space == std::string::npos || space + 1 == line.size())
                        throw std::runtime_error("Hidden dump path required");
                    const auto hidden = model.hidden();
                    std::ofstream out(line.substr(space + 1), std::ios::binary | std::ios::trunc);
                    if (!out) throw std::runtime_error("Cannot open hidden dump path");
                    out.write(reinterpret_cast<const char*>(hidden.data()), std::streamsize(hidden.size_bytes()));
                    out.close();
                    if (!out) throw std::runtime_error("Failed writing hidden dump");
                    std::cout << "{\"ok\":true,\"count\":" << hidden.size() << ",\"position\":" << model.position()
                              << ",\"format\":\"f32le\"}\n";
                } else if (command == "dump") {
                    const auto space = line.find(' ');
                    if (space == std::string::npos || space + 1 == line.size())
                        throw std::runtime_error("Dump path required");
                    const auto& logits = model.logits();
                    if (logits.size() != size_t(kV) || model.position() == 0)
                        throw std::runtime_error("No logits to dump");
                    std::ofstream out(line.substr(space + 1), std::ios::binary | std::ios::trunc);
                    if (!out) throw std::runtime_error("Cannot open dump path");
                    out.write(reinterpret_cast<const char*>(logits.data()), std::streamsize(logits.size() * 4));
                    out.close();
                    if (!out) throw std::runtime_error("Failed writing logits dump");
                    std::cout << "{\"ok\":true,\"count\":" << kV << ",\"position\":" << model.position() << "}\n";
                } else if (command == "stats") {
                    no_more(in);
                    handshake(options, model);
                    continue;
                } else {
                    throw std::runtime_error("Unknown command");
                }
            } catch (const std::exception& error) {
                // Any error resets model, history and sampler presence (engine/main.cpp:190-193).
                try {
                    model.reset();
                } catch (...) {
                }
                sampler.reset();
                history.clear();
                std::cout << "{\"error\":" << json_string(error.what()) << ",\"position\":0}\n";
            }
            std::cout << std::flush;
        }
        return 0;
    } catch (const std::exception& error) {
        std::cerr << "qwen_gpu: " << error.what() << '\n';
        return 1;
    }
}
