#pragma once
// Row-major [num_sequences][max_blocks_per_sequence] snapshot of page ids,
// short rows padded with invalid_block(), plus per-row token counts. Holds no
// references. Same surface as the reference's
// include/kvflux/v2/batch_block_table.h:12-36.

#include "kvflux/v2/sequence_state.h"

#include <cstddef>
#include <vector>

namespace kvflux::v2 {

class BatchBlockTable {
public:
    std::size_t num_sequences() const noexcept { return lengths_.size(); }
    std::size_t max_blocks_per_sequence() const noexcept { return width_; }
    const std::vector<PhysicalBlockID>& block_table() const noexcept { return table_; }
    const std::vector<std::size_t>& sequence_lengths() const noexcept { return lengths_; }
    static constexpr PhysicalBlockID invalid_block() noexcept {
        return static_cast<PhysicalBlockID>(-1);
    }

    // std::out_of_range outside the table or on padding.
    PhysicalBlockID physical_id(std::size_t request, std::size_t logical_block) const;

private:
    friend BatchBlockTable build_batch_block_table(const std::vector<const SequenceState*>&);
    std::size_t width_ = 0;
    std::vector<PhysicalBlockID> table_;
    std::vector<std::size_t> lengths_;
};

BatchBlockTable build_batch_block_table(const std::vector<const SequenceState*>& sequences);

} // namespace kvflux::v2
