// The per-layer key/value cache interface model code uses.
//
// Method names, parameters and meaning are the reference's
// (include/vvllm/kv_cache/kv_cache.h) so that transformer_forward
// (include/vvllm/model/transformer.h:145-160) drives a KVCacheHIP unchanged:
// init() sizes the cache once, append() writes num_tokens rows of kv_dim
// values for one layer at the current length, k()/v() return the layer's
// rows from position 0, advance() moves the length after all layers have
// appended, reset()/truncate() shorten it.
#pragma once

#include <cstddef>

namespace vvllm
{

class KVCache
{
public:
    virtual ~KVCache() = default;

    virtual void init(std::size_t num_layers, std::size_t kv_dim) = 0;
    virtual void append(std::size_t layer, const float* k, const float* v, std::size_t num_tokens) = 0;
    virtual const float* k(std::size_t layer) const = 0;
    virtual const float* v(std::size_t layer) const = 0;

    void advance(std::size_t num_tokens) { seq_len_ += num_tokens; }
    virtual void reset() = 0;
    virtual void truncate(std::size_t new_seq_len) = 0;

protected:
    std::size_t seq_len_ = 0;
    std::size_t kv_dim_ = 0;
};

}  // namespace vvllm
