// Converted-weights cache (the role of the reference's WeightCache,
// src/engine/weights.hip:26-164: record while converting, replay on the next
// load). File: a 64-byte head (magic, the caller's key, the layout version),
// then per piece a 16-byte record (byte count) and the bytes padded to 64,
// then the piece count. A file is replayed only when every record lies inside
// it and the count matches; it is written under "<path>.tmp" and renamed once
// complete, so an interrupted load never leaves a file that replays.
#include "wcache.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

namespace qwq4 {

namespace {
constexpr char MAGIC[8] = {'Q', 'W', 'Q', '4', 'T', 'I', 'L', 'E'};
size_t pad64(size_t b) { return (b + 63) / 64 * 64; }
}  // namespace

bool WCache::try_replay(const std::string &path, uint64_t key) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return false;
    struct stat sb;
    if (fstat(fd, &sb) != 0 || size_t(sb.st_size) < sizeof(Head) + sizeof(uint64_t)) {
        ::close(fd);
        return false;
    }
    const size_t size = size_t(sb.st_size);
    void *m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) return false;
    const uint8_t *p = static_cast<const uint8_t *>(m);
    Head h;
    std::memcpy(&h, p, sizeof h);
    bool ok = std::memcmp(h.magic, MAGIC, 8) == 0 && h.key == key && h.version == LAYOUT_VERSION;
    // walk the records: all inside the file, then the count
    size_t off = sizeof(Head);
    uint64_t n = 0;
    while (ok && off + sizeof(uint64_t) < size) {
        Piece pc;
        if (off + sizeof pc > size) {
            ok = false;
            break;
        }
        std::memcpy(&pc, p + off, sizeof pc);
        if (pc.bytes > size - off - sizeof pc) {
            ok = false;
            break;
        }
        off += sizeof pc + pad64(size_t(pc.bytes));
        ++n;
    }
    uint64_t count = ~0ull;
    if (ok && off + sizeof count == size) std::memcpy(&count, p + off, sizeof count);
    if (!ok || count != n) {
        munmap(m, size);
        return false;
    }
    map_ = p;
    size_ = size;
    off_ = sizeof(Head);
    total_ = n;
    return true;
}

void WCache::open(const std::string &path, uint64_t key, std::string &err) {
    path_ = path;
    if (try_replay(path, key)) {
        mode_ = REPLAY;
        return;
    }
    out_ = std::fopen((path + ".tmp").c_str(), "wb");
    if (!out_) {
        err = "cannot write " + path + ".tmp";
        return;
    }
    Head h{};
    std::memcpy(h.magic, MAGIC, 8);
    h.key = key;
    h.version = LAYOUT_VERSION;
    if (std::fwrite(&h, sizeof h, 1, out_) != 1) {
        std::fclose(out_);
        out_ = nullptr;
        std::remove((path + ".tmp").c_str());
        err = "cannot write " + path + ".tmp";
        return;
    }
    mode_ = RECORD;
}

WCache::~WCache() {
    if (map_) munmap(const_cast<uint8_t *>(map_), size_);
    if (out_) {  // never finished: the partial recording is dropped
        std::fclose(out_);
        std::remove((path_ + ".tmp").c_str());
    }
}

bool WCache::put(const void *host, size_t bytes, std::string &err) {
    if (mode_ != RECORD) return mode_ == OFF;
    static const uint8_t zeros[64] = {};
    const Piece pc{uint64_t(bytes), 0};
    bool ok = std::fwrite(&pc, sizeof pc, 1, out_) == 1 && (bytes == 0 || std::fwrite(host, bytes, 1, out_) == 1);
    ok = ok && (bytes % 64 == 0 || std::fwrite(zeros, 64 - bytes % 64, 1, out_) == 1);
    if (!ok) {
        std::fclose(out_);
        out_ = nullptr;
        std::remove((path_ + ".tmp").c_str());
        mode_ = OFF;
        err = "writing " + path_ + ".tmp failed; loading goes on without a cache";
        return false;
    }
    ++pieces_;
    return true;
}

const void *WCache::next(size_t bytes, std::string &err) {
    if (mode_ != REPLAY) {
        err = "not replaying a cache";
        return nullptr;
    }
    if (pieces_ >= total_) {
        err = path_ + ": more pieces asked for than the cache holds (delete it)";
        return nullptr;
    }
    Piece pc;
    std::memcpy(&pc, map_ + off_, sizeof pc);
    if (pc.bytes != bytes) {
        err = path_ + ": piece " + std::to_string(pieces_) + " holds " + std::to_string(pc.bytes) + " bytes, " +
              std::to_string(bytes) + " expected (delete it)";
        return nullptr;
    }
    const void *d = map_ + off_ + sizeof pc;
    off_ += sizeof pc + pad64(size_t(bytes));
    ++pieces_;
    return d;
}

bool WCache::finish(std::string &err) {
    if (mode_ == REPLAY) {
        if (pieces_ != total_) {
            err = path_ + ": " + std::to_string(total_ - pieces_) + " pieces left unused (delete it)";
            return false;
        }
        return true;
    }
    if (mode_ != RECORD) return true;
    const bool ok = std::fwrite(&pieces_, sizeof pieces_, 1, out_) == 1 && std::fflush(out_) == 0;
    std::fclose(out_);
    out_ = nullptr;
    if (ok && std::rename((path_ + ".tmp").c_str(), path_.c_str()) == 0) {
        mode_ = OFF;
        return true;
    }
    std::remove((path_ + ".tmp").c_str());
    mode_ = OFF;
    err = "could not complete " + path_;
    return false;
}

}  // namespace qwq4
