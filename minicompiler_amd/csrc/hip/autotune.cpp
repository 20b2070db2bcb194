#include "autotune.hpp"

#include "hip_rt.h"
#include "matmul.h"
#include "matmul_policy.hpp"

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdlib>
#include <fstream>
#include <map>
#include <mutex>
#include <set>
#include <sstream>
#include <tuple>

namespace minicompiler::hip {

namespace {

constexpr std::size_t kMaxWorkspace = std::size_t{512} << 20;

// (device tag, m, n, k) -> choice.
using Key = std::tuple<std::string, int, int, int>;

struct Decisions {
    std::mutex mu;
    std::map<Key, Fp32Choice> choice;
    std::set<std::string> loaded;  // device tags whose file has been read
};

Decisions& decisions() {
    static Decisions d;
    return d;
}

// "gfx950:sramecc+:xnack-" with 256 CUs -> "gfx950_sramecc_xnack_256cu".
std::string device_tag(const DeviceInfo& d) {
    std::string t;
    for (char c : d.arch) t += (c == ':' || c == '+' || c == '-') ? '_' : c;
    while (!t.empty() && t.back() == '_') t.pop_back();
    std::string out;
    for (char c : t) {
        if (c == '_' && !out.empty() && out.back() == '_') continue;
        out += c;
    }
    return out + "_" + std::to_string(d.cu_count) + "cu";
}

std::string decisions_file(const std::string& tag) {
    const char* dir = std::getenv("MINICOMPILER_HIP_CACHE_DIR");
    if (dir == nullptr || *dir == '\0') return {};
    return std::string(dir) + "/autotune_" + tag + ".txt";
}

// The file holds one decision per line: "m n k splits ring_cfg". Lines
// that do not parse, or name a choice outside the candidates, are ignored.
void load_file(Decisions& d, const std::string& tag, int cu_count) {
    if (!d.loaded.insert(tag).second) return;
    const std::string path = decisions_file(tag);
    if (path.empty()) return;
    std::ifstream f(path);
    std::string line;
    while (std::getline(f, line)) {
        std::istringstream s(line);
        int m = 0, n = 0, k = 0;
        Fp32Choice c;
        if (!(s >> m >> n >> k >> c.splits >> c.ring_cfg) || m < 1 || n < 1 || k < 1) continue;
        const std::vector<Fp32Choice> cands = autotune_candidates(m, n, k, cu_count);
        if (std::find(cands.begin(), cands.end(), c) == cands.end()) continue;
        d.choice[Key{tag, m, n, k}] = c;
    }
}

void append_file(const std::string& tag, int m, int n, int k, const Fp32Choice& c) {
    const std::string path = decisions_file(tag);
    if (path.empty()) return;
    std::ofstream f(path, std::ios::app);
    if (f) f << m << ' ' << n << ' ' << k << ' ' << c.splits << ' ' << c.ring_cfg << '\n';
}

struct DeviceMem {
    void* p = nullptr;
    DeviceMem() = default;
    DeviceMem(const DeviceMem&) = delete;
    DeviceMem& operator=(const DeviceMem&) = delete;
    ~DeviceMem() {
        if (p) mchip_free(p);
    }
};

struct Resources {
    void* stream = nullptr;
    void* start = nullptr;
    void* stop = nullptr;
    ~Resources() {
        if (start) mchip_event_destroy(start);
        if (stop) mchip_event_destroy(stop);
        if (stream) mchip_stream_destroy(stream);
    }
};

Status hip_status(int rc, const char* what) {
    if (rc == 0) return Status();
    return Error{std::string("autotune: ") + what + ": " + mchip_error_string(rc)};
}

#define MC_AT_TRY(call)                                     \
    do {                                                    \
        Status st_ = hip_status((call), #call);             \
        if (!st_.ok()) return st_.error();                  \
    } while (0)

Result<Fp32Choice> time_candidates(int m, int n, int k, const std::vector<Fp32Choice>& cands, bool fold) {
    const std::size_t mn = static_cast<std::size_t>(m) * n;
    int max_split = 1;
    for (const Fp32Choice& c : cands) max_split = std::max(max_split, c.splits);
    DeviceMem a, b, c, ws, counters;
    Resources r;
    MC_AT_TRY(mchip_malloc(&a.p, static_cast<std::size_t>(m) * k * 4));
    MC_AT_TRY(mchip_malloc(&b.p, static_cast<std::size_t>(k) * n * 4));
    MC_AT_TRY(mchip_malloc(&c.p, mn * 4));
    if (max_split > 1) MC_AT_TRY(mchip_malloc(&ws.p, static_cast<std::size_t>(max_split) * mn * 4));
    const std::size_t counter_bytes = static_cast<std::size_t>(mchip_split_counter_bytes(m, n));
    if (max_split > 1 && fold) {
        MC_AT_TRY(mchip_malloc(&counters.p, counter_bytes));
    }
    MC_AT_TRY(mchip_stream_create(&r.stream));
    MC_AT_TRY(mchip_event_create(&r.start));
    MC_AT_TRY(mchip_event_create(&r.stop));
    // Operands of ordinary magnitude (every float 0x3c3c3c3c, about 0.0115):
    // the matrix units draw power, and the clock follows, by the data.
    MC_AT_TRY(mchip_memset_async(a.p, 0x3c, static_cast<std::size_t>(m) * k * 4, r.stream));
    MC_AT_TRY(mchip_memset_async(b.p, 0x3c, static_cast<std::size_t>(k) * n * 4, r.stream));
    if (counters.p) MC_AT_TRY(mchip_memset_async(counters.p, 0, counter_bytes, r.stream));

    auto launch = [&](const Fp32Choice& ch) {
        const int s = ch.splits;
        const MatmulKernel kernel = s > 1 ? MatmulKernel::SplitK : MatmulKernel::DoubleBuffered;
        return mchip_launch_matmul_fold(static_cast<int>(kernel), static_cast<const float*>(a.p),
                                        static_cast<const float*>(b.p), static_cast<float*>(c.p), m, n, k, r.stream, s,
                                        s > 1 ? static_cast<float*>(ws.p) : nullptr, ch.ring_cfg,
                                        s > 1 ? static_cast<unsigned*>(counters.p) : nullptr);
    };
    auto time_reps = [&](const Fp32Choice& s, int reps, double* ms) -> Status {
        MC_AT_TRY(launch(s));
        MC_AT_TRY(mchip_event_record(r.start, r.stream));
        for (int i = 0; i < reps; ++i) MC_AT_TRY(launch(s));
        MC_AT_TRY(mchip_event_record(r.stop, r.stream));
        MC_AT_TRY(mchip_event_synchronize(r.stop));
        float total = 0.0f;
        MC_AT_TRY(mchip_event_elapsed_ms(&total, r.start, r.stop));
        *ms = static_cast<double>(total) / reps;
        return Status();
    };

    // Warm-up: the GPU raises its clock only under sustained load (tens of
    // milliseconds), and the first candidates would otherwise be timed cold.
    const auto until = std::chrono::steady_clock::now() + std::chrono::milliseconds(40);
    while (std::chrono::steady_clock::now() < until) {
        for (const Fp32Choice& s : cands) MC_AT_TRY(launch(s));
        MC_AT_TRY(mchip_stream_synchronize(r.stream));
    }
    // About a millisecond of launches per timing, best of three rounds.
    std::vector<int> reps(cands.size(), 2);
    std::vector<double> best(cands.size(), 1e30);
    for (std::size_t i = 0; i < cands.size(); ++i) {
        double ms = 0;
        Status st = time_reps(cands[i], 1, &ms);
        if (!st.ok()) return st.error();
        reps[i] = static_cast<int>(std::clamp(1.0 / std::max(ms, 1e-6), 2.0, 64.0));
    }
    for (int round = 0; round < 3; ++round) {
        for (std::size_t i = 0; i < cands.size(); ++i) {
            double ms = 0;
            Status st = time_reps(cands[i], reps[i], &ms);
            if (!st.ok()) return st.error();
            best[i] = std::min(best[i], ms);
        }
    }
    // The default comes first; another candidate has to be more than 2%
    // faster than the best before it to be chosen.
    std::size_t pick = 0;
    for (std::size_t i = 1; i < cands.size(); ++i) {
        if (best[i] < 0.98 * best[pick]) pick = i;
    }
    return cands[pick];
}

}  // namespace

std::vector<Fp32Choice> autotune_candidates(int m, int n, int k, int cu_count) {
    const int rule = m >= 1 && n >= 1 && k >= 1 && cu_count >= 1 ? split_k_splits(m, n, k, cu_count) : 1;
    std::vector<Fp32Choice> out{Fp32Choice{std::max(rule, 1), MCHIP_RING_NONE}};
    if (m < 1 || n < 1 || k < 1 || cu_count < 1 || k % 32 != 0 || n % 4 != 0) return out;
    auto tiles = [&](std::int64_t bm, std::int64_t bn) {
        return ((static_cast<std::int64_t>(m) + bm - 1) / bm) * ((static_cast<std::int64_t>(n) + bn - 1) / bn);
    };
    if (tiles(kSplitTileM, kSplitTileN) >= 2LL * cu_count) return out;
    const std::int64_t mn = static_cast<std::int64_t>(m) * n;
    const struct { int cfg; std::int64_t bm, bn; } cfgs[] = {
        {MCHIP_RING_WIDE, 128, 128}, {MCHIP_RING_MID, 64, 128}, {MCHIP_RING_THIN, 32, 128}};
    for (const auto& c : cfgs) {
        const std::int64_t t = tiles(c.bm, c.bn);
        for (int s = 1; s <= 64; s *= 2) {
            if (s > 1 && (s > k / 64 || t * s > 4LL * cu_count)) break;
            if (s > 1 && static_cast<std::size_t>(s) * static_cast<std::size_t>(mn) * 4 > kMaxWorkspace) break;
            const Fp32Choice ch{s, c.cfg};
            if (std::find(out.begin(), out.end(), ch) == out.end()) out.push_back(ch);
        }
    }
    return out;
}

Result<Fp32Choice> autotune_fp32(const DeviceInfo& device, int m, int n, int k, bool fold) {
    const std::vector<Fp32Choice> cands = autotune_candidates(m, n, k, device.cu_count);
    if (cands.size() == 1) return cands[0];
    const std::string tag = device_tag(device) + (fold ? "_fold" : "");
    Decisions& d = decisions();
    std::lock_guard<std::mutex> lock(d.mu);
    load_file(d, tag, device.cu_count);
    const Key key{tag, m, n, k};
    if (auto it = d.choice.find(key); it != d.choice.end()) return it->second;
    Result<Fp32Choice> chosen = time_candidates(m, n, k, cands, fold);
    if (!chosen.ok()) return chosen.error();
    d.choice[key] = chosen.value();
    append_file(tag, m, n, k, chosen.value());
    return chosen.value();
}

std::size_t autotune_cached_decisions() {
    Decisions& d = decisions();
    std::lock_guard<std::mutex> lock(d.mu);
    return d.choice.size();
}

}  // namespace minicompiler::hip
