// Dataset — the trainer's token source: flat little-endian uint32 token
// files (.bin), concatenated in file-name order, read as windows of T + 1
// tokens (input = tokens[p .. p+T-1], target = tokens[p+1 .. p+T]) with
// stride T per batch row, wrapping around the end of the data.
// Same API and batches as the reference's include/tensor/data/dataset.hpp
// (src/data/dataset.cpp:14-71).
#pragma once
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace tensor::data {

struct DataError : std::runtime_error {
    explicit DataError(const std::string& m) : std::runtime_error("DataError: " + m) {}
};

class Dataset {
public:
    // A .bin file, or every .bin file of a directory sorted by name.
    static Dataset load(const std::string& dir);

    // input_ids and target_ids, [B * T] int32 each.
    std::pair<std::vector<int32_t>, std::vector<int32_t>> next_batch(int B, int T);

    std::size_t total_tokens() const { return tokens_.size(); }
    std::size_t tokens_consumed() const { return consumed_; }

private:
    std::vector<uint32_t> tokens_;
    std::size_t pos_ = 0;
    std::size_t consumed_ = 0;
};

}  // namespace tensor::data
