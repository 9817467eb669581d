#pragma once
// Full-block prefix sharing on top of PhysicalBlockPool's publish/lookup.
// Same surface as the reference's include/kvflux/v2/prefix_cache.h:9-27.

#include "kvflux/v2/sequence_state.h"

namespace kvflux::v2 {

class PrefixCache {
public:
    explicit PrefixCache(PhysicalBlockPool& pool) noexcept : pool_(pool) {}

    // On an empty sequence, maps leading full blocks of `tokens` that are
    // published in the pool (stops at the first miss; a partial tail is never
    // shared). Returns the number of shared tokens. All-or-nothing on error.
    std::size_t attach_cached_prefix(SequenceState& sequence, const Tokens& tokens);

    // Publishes logical block `logical_block` of `sequence` under `prefix`
    // (the tokens from the start of the sequence to the end of that block),
    // after its K/V have been written and synchronised.
    void publish_computed_block(const SequenceState& sequence, std::size_t logical_block,
                                const Tokens& prefix);

private:
    PhysicalBlockPool& pool_;
};

} // namespace kvflux::v2
