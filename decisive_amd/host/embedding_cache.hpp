// embedding_cache.hpp -- the Rocm backend's Cache: packed embedding rows kept
// by token id, least recently used first out, under a byte budget.
//
// Restates EmbeddingCache of src/inference/browser/pplx.rs:45-138:
//  - keep(): a row larger than the whole budget is not kept; otherwise the
//    cache holds at most capacity / row_bytes rows, the touched id moves to
//    the back and the oldest ids leave from the front (:66-79);
//  - load(): duplicate ids in one request are read once; hits are served and
//    touched; misses are read in chunks of 8, with a cancellation check before
//    each chunk, and an incomplete row is an INVALID_CHECKPOINT (:80-137);
//  - the result is the rows of `ids` in request order, duplicates repeated.
// The budget covers reusable rows only (the reference's readme.md:25), not
// weights or device scratch.
#pragma once

#include <cstdint>
#include <deque>
#include <functional>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "inference.hpp"

namespace decisive {

class EmbeddingCache {
public:
    // Reads the packed rows of `ids` (in that order, concatenated).
    using Reader = std::function<Result<std::vector<uint8_t>>(const std::vector<uint32_t> &ids)>;

    explicit EmbeddingCache(size_t capacity = 0) : capacity_(capacity) {}

    void clear() {
        entries_.clear();
        order_.clear();
    }
    size_t capacity() const { return capacity_; }
    size_t rows() const { return entries_.size(); }
    bool contains(uint32_t id) const { return entries_.count(id) != 0; }
    const std::deque<uint32_t> &order() const { return order_; }
    // Rows served from the cache / read through the reader, over the cache's life.
    uint64_t hits() const { return hits_; }
    uint64_t misses() const { return misses_; }

    Result<std::vector<uint8_t>> load(const std::vector<uint32_t> &ids, const Reader &reader, size_t row_bytes,
                                      const Cancellation &cancellation) {
        std::unordered_map<uint32_t, std::vector<uint8_t>> selected;
        std::vector<uint32_t> missing;
        std::unordered_set<uint32_t> seen_missing;
        for (uint32_t id : ids) {
            if (selected.count(id) || seen_missing.count(id)) continue;
            auto it = entries_.find(id);
            if (it != entries_.end()) {
                std::vector<uint8_t> bytes = it->second;
                selected[id] = bytes;
                keep(id, std::move(bytes));
                hits_++;
            } else {
                missing.push_back(id);
                seen_missing.insert(id);
            }
        }
        for (size_t at = 0; at < missing.size(); at += kChunk) {
            Status s = cancellation.check();
            if (!s) return s.error();
            std::vector<uint32_t> chunk(missing.begin() + at,
                                        missing.begin() + std::min(missing.size(), at + kChunk));
            auto read = reader(chunk);
            if (!read) return read.error();
            const std::vector<uint8_t> &bytes = read.value();
            if (bytes.size() != chunk.size() * row_bytes)
                return Error("INVALID_CHECKPOINT", "Incomplete embedding row");
            for (size_t i = 0; i < chunk.size(); i++) {
                std::vector<uint8_t> row(bytes.begin() + i * row_bytes, bytes.begin() + (i + 1) * row_bytes);
                selected[chunk[i]] = row;
                keep(chunk[i], std::move(row));
                misses_++;
            }
        }
        std::vector<uint8_t> rows;
        rows.reserve(ids.size() * row_bytes);
        for (uint32_t id : ids) {
            const auto &r = selected[id];
            rows.insert(rows.end(), r.begin(), r.end());
        }
        return rows;
    }

private:
    static constexpr size_t kChunk = 8;

    void keep(uint32_t id, std::vector<uint8_t> bytes) {
        if (bytes.empty() || bytes.size() > capacity_) return;
        const size_t limit = capacity_ / bytes.size();
        for (auto it = order_.begin(); it != order_.end();) {
            if (*it == id) it = order_.erase(it);
            else ++it;
        }
        order_.push_back(id);
        entries_[id] = std::move(bytes);
        while (order_.size() > limit) {
            entries_.erase(order_.front());
            order_.pop_front();
        }
    }

    size_t capacity_;
    std::unordered_map<uint32_t, std::vector<uint8_t>> entries_;
    std::deque<uint32_t> order_;
    uint64_t hits_ = 0, misses_ = 0;
};

}  // namespace decisive
