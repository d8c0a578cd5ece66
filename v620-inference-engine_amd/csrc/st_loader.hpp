// Safetensors file access for the q4 weight loader (host side).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace qwq4 {

struct StTensor {
    std::string name, dtype;        // dtype as the header writes it: "I32", "BF16", "F16", ...
    std::vector<int64_t> shape;
    const uint8_t *data = nullptr;  // inside the mapping
    size_t nbytes = 0;
};

class StFile {
public:
    bool open(const std::string &path, std::string &err);
    ~StFile();
    const StTensor *find(const std::string &name) const;
    const std::map<std::string, StTensor> &tensors() const { return index_; }

private:
    std::string path_;
    const uint8_t *data_ = nullptr;
    size_t size_ = 0;
    std::map<std::string, StTensor> index_;  // ordered: a stable listing
};

}  // namespace qwq4
