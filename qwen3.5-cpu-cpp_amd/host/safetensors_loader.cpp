// Safetensors reader: mmap each shard, parse its JSON tensor table with a small
// recursive-descent scanner, keep (dtype, shape, offset, size) per tensor name.
// Error messages and return conventions follow src/safetensors_loader.cpp:131-298.
#include "safetensors_loader.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdlib>
#include <filesystem>
#include <iostream>
#include <system_error>

namespace {

class HeaderScanner {
public:
    HeaderScanner(const char* p, const char* e) : p_(p), e_(e) {}
    bool ok() const { return ok_; }

    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }
    bool peek(char c) {
        ws();
        return p_ < e_ && *p_ == c;
    }
    bool take(char c) {
        if (peek(c)) {
            ++p_;
            return true;
        }
        ok_ = false;
        return false;
    }
    bool take_if(char c) {
        if (peek(c)) {
            ++p_;
            return true;
        }
        return false;
    }
    std::string str() {
        std::string out;
        if (!take('"')) return out;
        while (p_ < e_ && *p_ != '"') {
            char c = *p_++;
            if (c == '\\' && p_ < e_) {
                const char n = *p_++;
                c = n == 'n' ? '\n' : n == 't' ? '\t' : n;
            }
            out.push_back(c);
        }
        if (p_ >= e_) {
            ok_ = false;
            return out;
        }
        ++p_;
        return out;
    }
    int64_t integer() {
        ws();
        const char* first = p_;
        if (p_ < e_ && (*p_ == '-' || *p_ == '+')) ++p_;
        while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        if (p_ == first) {
            ok_ = false;
            return 0;
        }
        return std::strtoll(std::string(first, p_).c_str(), nullptr, 10);
    }
    std::vector<int64_t> int_list() {
        std::vector<int64_t> v;
        if (!take('[')) return v;
        if (take_if(']')) return v;
        do {
            v.push_back(integer());
        } while (ok_ && take_if(','));
        take(']');
        return v;
    }
    void skip() {
        ws();
        if (p_ >= e_) {
            ok_ = false;
            return;
        }
        const char c = *p_;
        if (c == '"') {
            str();
        } else if (c == '{' || c == '[') {
            const char close = c == '{' ? '}' : ']';
            ++p_;
            if (take_if(close)) return;
            do {
                if (c == '{') {
                    str();
                    take(':');
                }
                skip();
            } while (ok_ && take_if(','));
            take(close);
        } else {
            while (p_ < e_ && *p_ != ',' && *p_ != '}' && *p_ != ']') ++p_;
        }
    }

private:
    const char* p_;
    const char* e_;
    bool ok_ = true;
};

}  // namespace

int64_t SafeTensors::Entry::numel() const {
    if (shape.empty()) return 0;
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
}

SafeTensors::~SafeTensors() { release(); }

void SafeTensors::release() {
    for (Shard& s : shards_)
        if (s.map) munmap(s.map, s.size);
    shards_.clear();
    entries_.clear();
    f32_cache_.clear();
}

bool SafeTensors::parse_shard(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) {
        std::cerr << "[safetensors] cannot open '" << path << "'\n";
        return false;
    }
    struct stat sb {};
    ::fstat(fd, &sb);
    const size_t size = static_cast<size_t>(sb.st_size);
    if (size < 8) {
        ::close(fd);
        std::cerr << "[safetensors] file too small\n";
        return false;
    }
    void* map = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map == MAP_FAILED) {
        std::cerr << "[safetensors] read failed\n";
        return false;
    }
    const int shard = static_cast<int>(shards_.size());
    shards_.push_back({map, size});
    const auto* bytes = static_cast<const uint8_t*>(map);

    uint64_t header_len = 0;
    std::memcpy(&header_len, bytes, 8);
    if (header_len > size - 8) {
        std::cerr << "[safetensors] header length exceeds file\n";
        return false;
    }
    const size_t data_base = 8 + static_cast<size_t>(header_len);
    HeaderScanner sc(reinterpret_cast<const char*>(bytes) + 8,
                     reinterpret_cast<const char*>(bytes) + data_base);
    if (!sc.take('{')) {
        std::cerr << "[safetensors] bad header\n";
        return false;
    }
    if (sc.take_if('}')) return true;
    do {
        std::string key = sc.str();
        sc.take(':');
        if (!sc.ok()) break;
        if (key == "__metadata__") {
            sc.skip();
            continue;
        }
        Entry e;
        int64_t off0 = 0, off1 = 0;
        sc.take('{');
        do {
            const std::string field = sc.str();
            sc.take(':');
            if (field == "dtype") {
                e.dtype = sc.str();
            } else if (field == "shape") {
                e.shape = sc.int_list();
            } else if (field == "data_offsets") {
                const std::vector<int64_t> v = sc.int_list();
                if (v.size() == 2) {
                    off0 = v[0];
                    off1 = v[1];
                }
            } else {
                sc.skip();
            }
        } while (sc.ok() && sc.take_if(','));
        sc.take('}');
        if (off0 < 0 || off1 < off0 || data_base + static_cast<size_t>(off1) > size) {
            std::cerr << "[safetensors] tensor '" << key << "' out of range\n";
            return false;
        }
        e.shard = shard;
        e.abs_offset = data_base + static_cast<size_t>(off0);
        e.nbytes = static_cast<size_t>(off1 - off0);
        entries_.emplace(std::move(key), std::move(e));
    } while (sc.ok() && sc.take_if(','));
    sc.take('}');
    if (!sc.ok()) {
        std::cerr << "[safetensors] header parse error\n";
        return false;
    }
    std::cerr << "[safetensors] shard '" << path << "': " << (size / (1024 * 1024)) << " MB\n";
    return true;
}

bool SafeTensors::load(const std::string& path) {
    release();
    return parse_shard(path);
}

bool SafeTensors::load_model(const std::string& model_dir) {
    release();
    std::vector<std::string> files;
    std::error_code ec;
    for (const auto& de : std::filesystem::directory_iterator(model_dir, ec))
        if (de.path().extension() == ".safetensors") files.push_back(de.path().string());
    if (files.empty()) {
        std::cerr << "[safetensors] no .safetensors files in '" << model_dir << "'\n";
        return false;
    }
    std::sort(files.begin(), files.end());
    for (const std::string& f : files)
        if (!parse_shard(f)) return false;
    std::cerr << "[safetensors] " << files.size() << " shard(s), " << entries_.size()
              << " tensors\n";
    return true;
}

const SafeTensors::Entry* SafeTensors::find(const std::string& name) const {
    const auto it = entries_.find(name);
    return it == entries_.end() ? nullptr : &it->second;
}

const void* SafeTensors::data(const std::string& name) const {
    const Entry* e = find(name);
    if (!e) return nullptr;
    return static_cast<const uint8_t*>(shards_[e->shard].map) + e->abs_offset;
}

WeightView SafeTensors::view(const std::string& name) const {
    WeightView v;
    const Entry* e = find(name);
    if (!e) return v;
    const void* p = data(name);
    v.numel = e->numel();
    if (e->dtype == "BF16") v.bf16 = static_cast<const uint16_t*>(p);
    else if (e->dtype == "F32") v.f32 = static_cast<const float*>(p);
    return v;
}

const float* SafeTensors::get_f32(const std::string& name, int64_t* out_numel) {
    const auto hit = f32_cache_.find(name);
    if (hit != f32_cache_.end()) {
        if (out_numel) *out_numel = static_cast<int64_t>(hit->second.size());
        return hit->second.data();
    }
    const Entry* e = find(name);
    if (!e) return nullptr;
    const int64_t n = e->numel();
    std::vector<float> buf(static_cast<size_t>(n));
    const void* src = data(name);
    if (e->dtype == "F32") {
        std::memcpy(buf.data(), src, static_cast<size_t>(n) * 4);
    } else if (e->dtype == "BF16") {
        const auto* s = static_cast<const uint16_t*>(src);
        for (int64_t i = 0; i < n; ++i) buf[static_cast<size_t>(i)] = bf16_to_f32(s[i]);
    } else {
        std::cerr << "[safetensors] unsupported dtype " << e->dtype << " for '" << name << "'\n";
        return nullptr;
    }
    auto res = f32_cache_.emplace(name, std::move(buf));
    if (out_numel) *out_numel = static_cast<int64_t>(res.first->second.size());
    return res.first->second.data();
}

bool SafeTensors::get_row_f32(const std::string& name, int64_t row, float* dst) const {
    const Entry* e = find(name);
    if (!e || e->shape.size() != 2) return false;
    const int64_t rows = e->shape[0], cols = e->shape[1];
    if (row < 0 || row >= rows) return false;
    const void* base = data(name);
    if (e->dtype == "F32") {
        std::memcpy(dst, static_cast<const float*>(base) + row * cols, static_cast<size_t>(cols) * 4);
    } else if (e->dtype == "BF16") {
        const uint16_t* s = static_cast<const uint16_t*>(base) + row * cols;
        for (int64_t i = 0; i < cols; ++i) dst[i] = bf16_to_f32(s[i]);
    } else {
        return false;
    }
    return true;
}
