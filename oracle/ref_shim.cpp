// extern "C" entry points over the reference's own CPU library, compiled from
// the reference sources in place (see oracle/Makefile, target `ref`). Used
// only by tests/golden/gen_golden.py and the CPU tests that cross-check the
// oracle; TEST INFRASTRUCTURE ONLY, never shipped or linked by the product.
//
// ref_reference_attention wraps kvflux::v2::reference_attention
// (reference src/v2/reference_attention.cpp:28-91).
// ref_run_trace interprets a small op language against the reference's
// PhysicalBlockPool / SequenceState / slot mapping / tables, so the same
// trace can be replayed on this repository's implementation.
#include "kvflux/physical_block_pool.h"
#include "kvflux/v2/batch_block_table.h"
#include "kvflux/v2/paged_kv_read.h"
#include "kvflux/v2/prefix_cache.h"
#include "kvflux/v2/reference_attention.h"
#include "kvflux/v2/sequence_state.h"
#include "kvflux/v2/slot_mapping.h"

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <vector>

namespace {

int status_of(const std::exception_ptr& e) {
    try {
        std::rethrow_exception(e);
    } catch (const kvflux::CapacityError&) {
        return -4;
    } catch (const std::invalid_argument&) {
        return -1;
    } catch (const std::out_of_range&) {
        return -2;
    } catch (const std::overflow_error&) {
        return -3;
    } catch (const std::logic_error&) {
        return -5;
    } catch (...) {
        return -9;
    }
}

} // namespace

extern "C" int ref_reference_attention(const float* q, std::size_t nq, const float* k,
                                       std::size_t nk, const float* v, std::size_t nv,
                                       std::size_t q_tokens, std::size_t kv_tokens,
                                       std::size_t q_heads, std::size_t kv_heads,
                                       std::size_t head_size, float* out) {
    try {
        const auto result = kvflux::v2::reference_attention(
            std::vector<float>(q, q + nq), std::vector<float>(k, k + nk),
            std::vector<float>(v, v + nv), {q_tokens, kv_tokens, q_heads, kv_heads, head_size});
        for (std::size_t i = 0; i < result.size(); ++i) out[i] = result[i];
        return 0;
    } catch (...) {
        return status_of(std::current_exception());
    }
}

// Trace ops (each op is 3 int64: code, a, b). Results are appended to `out`
// (capacity `out_cap`); returns the number written or -100 on overflow.
//   0 ALLOC            -> page id                (handle kept in list H)
//   1 FREE h           -> 0 / error
//   2 RETAIN h         -> 0 / error
//   3 NEW_SEQ          -> sequence index         (list S)
//   4 APPEND s n       -> 0 / error
//   5 APPEND_ONE s     -> page * 2^20 + offset / error
//   6 FORK s           -> new sequence index / error
//   7 DROP s           -> 0
//   8 SLOT s pos       -> slot / error
//   9 TABLE s          -> count, then each page id
//  10 AVAILABLE        -> pool.available()
//  11 REFS s logical   -> ref count / error
//  12 APPEND_COW s     -> page * 2^20 + offset / error (no-op copier)
//  13 BATCH n          -> over the last n live sequences: width, lengths..., table...
//  14 PUBLISH s blk    -> 0 / error (prefix = tokens 0..(blk+1)*bs-1, token = index)
//  15 ATTACH s ntok    -> shared tokens / error (prefix tokens = index)
//  16 ID h             -> pool.id(handle) / error
extern "C" long ref_run_trace(std::size_t capacity, std::size_t block_size, const long* ops,
                              std::size_t num_ops, long* out, std::size_t out_cap) {
    using namespace kvflux;
    using namespace kvflux::v2;
    PhysicalBlockPool pool(capacity, block_size);
    PrefixCache cache(pool);
    std::vector<PhysicalBlockHandle> handles;
    std::vector<std::unique_ptr<SequenceState>> seqs;
    std::size_t n = 0;
    auto emit = [&](long value) {
        if (n < out_cap) out[n] = value;
        ++n;
    };
    auto seq = [&](long i) -> SequenceState& {
        if (i < 0 || static_cast<std::size_t>(i) >= seqs.size() || !seqs[i]) {
            throw std::runtime_error("bad trace sequence index");
        }
        return *seqs[i];
    };
    auto tokens = [](std::size_t count) {
        Tokens t(count);
        for (std::size_t i = 0; i < count; ++i) t[i] = static_cast<Token>(i);
        return t;
    };
    for (std::size_t i = 0; i < num_ops; ++i) {
        const long code = ops[3 * i], a = ops[3 * i + 1], b = ops[3 * i + 2];
        try {
            switch (code) {
            case 0: {
                handles.push_back(pool.allocate());
                emit(static_cast<long>(handles.back().id));
                break;
            }
            case 1: pool.free(handles.at(a)); emit(0); break;
            case 2: pool.retain(handles.at(a)); emit(0); break;
            case 3: seqs.push_back(std::make_unique<SequenceState>(seqs.size(), pool));
                    emit(static_cast<long>(seqs.size() - 1)); break;
            case 4: seq(a).append_tokens(static_cast<std::size_t>(b)); emit(0); break;
            case 5: {
                const auto loc = seq(a).append_token();
                emit(static_cast<long>(loc.physical_block * (1L << 20) + loc.offset_in_block));
                break;
            }
            case 6: {
                auto fork = std::make_unique<SequenceState>(seq(a).fork_shared(seqs.size()));
                seqs.push_back(std::move(fork));
                emit(static_cast<long>(seqs.size() - 1));
                break;
            }
            case 7: seqs.at(a).reset(); emit(0); break;
            case 8: {
                const auto slots = build_slot_mapping({{&seq(a), static_cast<std::size_t>(b)}});
                emit(static_cast<long>(slots.at(0)));
                break;
            }
            case 9: {
                const auto table = build_read_block_table(seq(a));
                emit(static_cast<long>(table.size()));
                for (auto id : table) emit(static_cast<long>(id));
                break;
            }
            case 10: emit(static_cast<long>(pool.available())); break;
            case 11: emit(static_cast<long>(seq(a).block_table().ref_count(static_cast<std::size_t>(b)))); break;
            case 12: {
                const auto loc = seq(a).append_token_with_copy([](auto, auto) {});
                emit(static_cast<long>(loc.physical_block * (1L << 20) + loc.offset_in_block));
                break;
            }
            case 13: {
                std::vector<const SequenceState*> batch;
                for (std::size_t j = seqs.size(); j-- > 0 && batch.size() < static_cast<std::size_t>(a);) {
                    if (seqs[j]) batch.insert(batch.begin(), seqs[j].get());
                }
                const auto t = build_batch_block_table(batch);
                emit(static_cast<long>(t.max_blocks_per_sequence()));
                for (auto l : t.sequence_lengths()) emit(static_cast<long>(l));
                for (auto id : t.block_table()) emit(static_cast<long>(id));
                break;
            }
            case 14: cache.publish_computed_block(seq(a), static_cast<std::size_t>(b),
                                                  tokens((b + 1) * block_size));
                     emit(0); break;
            case 15: emit(static_cast<long>(cache.attach_cached_prefix(seq(a), tokens(b)))); break;
            case 16: emit(static_cast<long>(pool.id(handles.at(a)))); break;
            default: emit(-99); break;
            }
        } catch (...) {
            emit(status_of(std::current_exception()));
        }
    }
    return n <= out_cap ? static_cast<long>(n) : -100;
}
