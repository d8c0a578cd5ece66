// Converted-weights cache (host side): the device buffers a loader fills, in
// the order it fills them, kept in one file so that a later load uploads them
// without reading or converting the checkpoint again.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <string>

namespace qwq4 {

class WCache {
public:
    enum Mode { OFF = 0, RECORD = 1, REPLAY = 2 };
    // Replays `path` when it is a complete cache written with this key and
    // layout version; otherwise records into "<path>.tmp" (renamed to path by
    // finish). When neither is possible the mode is OFF and err says why.
    void open(const std::string &path, uint64_t key, std::string &err);
    ~WCache();
    Mode mode() const { return mode_; }
    // RECORD: appends one piece of `bytes` bytes (a write error drops the
    // recording: mode OFF, err set, the load goes on without a cache).
    bool put(const void *host, size_t bytes, std::string &err);
    // REPLAY: the next piece, which must hold exactly `bytes` bytes; a pointer
    // into the mapping, or null with err set.
    const void *next(size_t bytes, std::string &err);
    // RECORD: completes the file and renames it into place. REPLAY: checks
    // that every piece was used.
    bool finish(std::string &err);
    uint64_t pieces() const { return pieces_; }

    static constexpr uint64_t LAYOUT_VERSION = 1;  // bump when the tiled layout changes

private:
    struct Head {
        char magic[8];
        uint64_t key, version, reserved[5];
    };
    struct Piece {
        uint64_t bytes, reserved;
    };
    static_assert(sizeof(Head) == 64 && sizeof(Piece) == 16, "cache header sizes");
    bool try_replay(const std::string &path, uint64_t key);

    Mode mode_ = OFF;
    std::string path_;
    std::FILE *out_ = nullptr;
    const uint8_t *map_ = nullptr;
    size_t size_ = 0, off_ = 0;
    uint64_t pieces_ = 0, total_ = 0;
};

}  // namespace qwq4
