#include "kernel_compiler.hpp"

#include "hip_rt.h"

#include <fcntl.h>
#include <unistd.h>

#include <atomic>
#include <cerrno>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <sstream>
#include <thread>

namespace minicompiler::hip {

namespace {

std::uint64_t fnv1a64(const std::string& s) {
    std::uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 0x100000001b3ull;
    }
    return h;
}

std::string disk_cache_path(const std::string& key) {
    const char* dir = std::getenv("MINICOMPILER_HIP_CACHE_DIR");
    if (dir == nullptr || *dir == '\0') return {};
    char name[64];
    std::snprintf(name, sizeof name, "/mc_%016llx.co", static_cast<unsigned long long>(fnv1a64(key)));
    return std::string(dir) + name;
}

bool read_file(const std::string& path, std::string* out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    std::ostringstream s;
    s << f.rdbuf();
    *out = s.str();
    return !out->empty();
}

// A cache file: the magic line; the key's length in decimal and a newline;
// the key itself; the code object's length in decimal, a space, its FNV-1a
// hash in hex and a newline; then the code object. A file whose key differs
// from the requested one (a hash collision, or a key from another compiler)
// or whose code does not have the recorded length and hash (a torn or
// truncated write) is a miss: the kernel is compiled again.
constexpr const char* kCacheMagic = "minicompiler-hip code object v2\n";

std::string hex64(std::uint64_t v) {
    char buf[17];
    std::snprintf(buf, sizeof buf, "%016llx", static_cast<unsigned long long>(v));
    return buf;
}

std::string cache_file_contents(const std::string& key, const std::string& code) {
    return std::string(kCacheMagic) + std::to_string(key.size()) + '\n' + key + std::to_string(code.size()) + ' ' +
           hex64(fnv1a64(code)) + '\n' + code;
}

bool all_digits(const std::string& s) { return !s.empty() && s.find_first_not_of("0123456789") == std::string::npos; }

bool code_from_cache_file(const std::string& file, const std::string& key, std::string* code) {
    const std::string magic(kCacheMagic);
    if (file.compare(0, magic.size(), magic) != 0) return false;
    const std::size_t nl = file.find('\n', magic.size());
    if (nl == std::string::npos) return false;
    const std::string len_text = file.substr(magic.size(), nl - magic.size());
    if (!all_digits(len_text) || len_text.size() > 18) return false;
    const std::size_t len = std::stoull(len_text);
    if (len != key.size() || file.size() <= nl + 1 + len || file.compare(nl + 1, len, key) != 0) return false;
    const std::size_t head = nl + 1 + len;
    const std::size_t nl2 = file.find('\n', head);
    const std::size_t sp = file.find(' ', head);
    if (nl2 == std::string::npos || sp == std::string::npos || sp > nl2) return false;
    const std::string code_len = file.substr(head, sp - head);
    if (!all_digits(code_len) || code_len.size() > 18) return false;
    const std::size_t clen = std::stoull(code_len);
    if (file.size() - (nl2 + 1) != clen || clen == 0) return false;
    std::string body = file.substr(nl2 + 1);
    if (file.compare(sp + 1, nl2 - sp - 1, hex64(fnv1a64(body))) != 0) return false;
    *code = std::move(body);
    return true;
}

// Writes `data` to a temporary file of a name no other writer uses (this
// process's id, a per-process counter and the thread's id, created with
// O_EXCL), then renames it over `path`: readers see the old file or the
// whole new one. Any failure leaves `path` alone.
void write_file_atomically(const std::string& path, const std::string& data) {
    static std::atomic<unsigned long long> counter{0};
    const std::string tmp = path + ".tmp." + std::to_string(static_cast<long long>(getpid())) + '.' +
                            std::to_string(counter.fetch_add(1)) + '.' +
                            hex64(std::hash<std::thread::id>{}(std::this_thread::get_id()));
    const int fd = open(tmp.c_str(), O_WRONLY | O_CREAT | O_EXCL | O_CLOEXEC, 0644);
    if (fd < 0) return;
    std::size_t done = 0;
    while (done < data.size()) {
        const ssize_t w = write(fd, data.data() + done, data.size() - done);
        if (w < 0 && errno == EINTR) continue;
        if (w <= 0) break;
        done += static_cast<std::size_t>(w);
    }
    const bool ok = close(fd) == 0 && done == data.size();
    if (!ok || std::rename(tmp.c_str(), path.c_str()) != 0) unlink(tmp.c_str());
}

std::string cache_key(const std::string& arch, const std::string& source) {
    int major = 0, minor = 0;
    mchip_rtc_version(&major, &minor);
    std::string key = "hiprtc " + std::to_string(major) + "." + std::to_string(minor) + '\n' + arch;
    for (const std::string& o : KernelCompiler::options_for(arch)) key += '\n' + o;
    return key + '\n' + source;
}

}  // namespace

KernelCompiler& KernelCompiler::instance() {
    static KernelCompiler compiler;
    return compiler;
}

std::vector<std::string> KernelCompiler::options_for(const std::string& arch) {
    return {"--offload-arch=" + arch, "-O3", "-std=c++17", "-ffp-contract=off",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
}

Result<std::string> KernelCompiler::compile_code_object(const std::string& source, const std::string& arch,
                                                        double* compile_ms) {
    const auto t0 = std::chrono::steady_clock::now();
    const std::string key = cache_key(arch, source);
    const std::string path = disk_cache_path(key);
    std::string code;
    std::string file;
    if (!path.empty() && read_file(path, &file) && code_from_cache_file(file, key, &code)) {
        if (compile_ms) *compile_ms = 0.0;
        return code;
    }
    const std::vector<std::string> opts = options_for(arch);
    std::vector<const char*> argv;
    for (const std::string& o : opts) argv.push_back(o.c_str());
    char* image = nullptr;
    char* log = nullptr;
    std::size_t size = 0;
    const int rc = mchip_rtc_compile(source.c_str(), "mc_generated.hip", argv.data(), static_cast<int>(argv.size()),
                                     &image, &size, &log);
    const std::string log_text = log ? log : "";
    mchip_rtc_free(log);
    if (rc != 0) {
        mchip_rtc_free(image);
        return Error{std::string("hipRTC could not compile a generated kernel (") + mchip_rtc_error_string(rc) +
                     "):\n" + log_text + "\n" + source};
    }
    code.assign(image, size);
    mchip_rtc_free(image);
    if (!path.empty()) write_file_atomically(path, cache_file_contents(key, code));
    if (compile_ms) {
        *compile_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    }
    return code;
}

Result<CompiledKernel> KernelCompiler::get(const std::string& source, const char* name, const std::string& arch,
                                           int device, double* compile_ms) {
    if (compile_ms) *compile_ms = 0.0;
    const std::string module_key = std::to_string(device) + '\n' + cache_key(arch, source);
    const std::string key = module_key + '\n' + name;
    void* module = nullptr;
    {
        std::lock_guard<std::mutex> lock(mutex_);
        const auto it = loaded_.find(key);
        if (it != loaded_.end()) return it->second;
        const auto m = modules_.find(module_key);
        if (m != modules_.end()) module = m->second;
    }
    if (module == nullptr) {
        // Compile outside the lock so executables can build kernels concurrently.
        Result<std::string> code = compile_code_object(source, arch, compile_ms);
        if (!code.ok()) return code.error();
        std::lock_guard<std::mutex> lock(mutex_);
        const auto m = modules_.find(module_key);
        if (m != modules_.end()) {
            module = m->second;
        } else {
            const int rc = mchip_module_load(&module, code->data());
            if (rc != 0) return Error{std::string("hipModuleLoadData: ") + mchip_error_string(rc)};
            modules_.emplace(module_key, module);
        }
    }
    std::lock_guard<std::mutex> lock(mutex_);
    const auto it = loaded_.find(key);
    if (it != loaded_.end()) return it->second;
    CompiledKernel k;
    k.module = module;
    const int rc = mchip_module_function(&k.function, module, name);
    if (rc != 0) return Error{std::string("hipModuleGetFunction(") + name + "): " + mchip_error_string(rc)};
    loaded_.emplace(key, k);
    return k;
}

}  // namespace minicompiler::hip
