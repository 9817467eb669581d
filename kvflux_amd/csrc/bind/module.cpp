// Python binding of the kvflux::v2 C++ layer (tests, benchmark, smoke run).
// Device pointers cross as Python ints; 0 is the null pointer.
// Exception mapping: std::invalid_argument -> ValueError,
// std::out_of_range -> IndexError, std::overflow_error -> OverflowError,
// kvflux::CapacityError -> CapacityError(RuntimeError), other
// std::logic_error -> LogicError(RuntimeError), std::runtime_error -> RuntimeError.
#include <pybind11/functional.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include "kvflux/v2/batch_block_table.h"
#include "kvflux/v2/copy_on_write.h"
#include "kvflux/v2/device_batch_table.h"
#include "kvflux/v2/prefix_cache.h"
#include "kvflux/v2/sequence_lifecycle.h"
#include "kvflux/v2/paged_attention.h"
#include "kvflux/v2/paged_kv_read.h"
#include "kvflux/v2/paged_kv_write.h"
#include "kvflux/v2/reference_attention.h"
#include "kvflux/v3/cache_directory.h"
#include "kvflux/v3/gpu_chunk_store.h"
#include "kvflux/v3/gpu_cpu_transfer.h"
#include "kvflux/v3/pinned_chunk_pool.h"

#include <chrono>
#include <cstdint>
#include <stdexcept>

namespace py = pybind11;
using kvflux::BlockHandle;
using kvflux::BlockManager;
using kvflux::CapacityError;
using kvflux::DType;
using kvflux::KVKind;
using kvflux::PhysicalBlockHandle;
using kvflux::PhysicalBlockPool;
using kvflux::Tokens;
using namespace kvflux::v2;

namespace {

void* ptr(std::uintptr_t address) { return reinterpret_cast<void*>(address); }
std::uintptr_t addr(const void* p) { return reinterpret_cast<std::uintptr_t>(p); }

} // namespace

// Seconds per call of `fn` over `reps` back-to-back calls, timed in C++ (no
// Python or argument conversion inside the timed loop).
template <typename Fn>
static double seconds_per_call(std::size_t reps, Fn&& fn) {
    if (reps == 0) throw std::invalid_argument("reps must be positive");
    const auto t0 = std::chrono::steady_clock::now();
    for (std::size_t i = 0; i < reps; ++i) fn();
    const std::chrono::duration<double> dt = std::chrono::steady_clock::now() - t0;
    return dt.count() / static_cast<double>(reps);
}

// Timing loops over the synchronous C++ API, for the benchmark: what a C++
// caller of the drop-in API pays per call (validation, metadata upload,
// launch, stream synchronisation).
static void bind_timing(py::module_ t) {
    t.def("write_paged_kv", [](PagedKVStorage& s, std::uintptr_t k, std::uintptr_t v, const SlotMapping& slots,
                               std::size_t reps) {
        py::gil_scoped_release release;
        return seconds_per_call(reps, [&] { write_paged_kv(s, ptr(k), ptr(v), slots); });
    });
    t.def("read_paged_kv_batch", [](const PagedKVStorage& s, const std::vector<const SequenceState*>& seqs,
                                    std::uintptr_t k, std::uintptr_t v, std::size_t reps) {
        py::gil_scoped_release release;
        return seconds_per_call(reps, [&] { read_paged_kv_batch(s, seqs, ptr(k), ptr(v)); });
    });
    t.def("paged_attention", [](const PagedKVStorage& s, const std::vector<const SequenceState*>& seqs,
                                const std::vector<std::uintptr_t>& q, const std::vector<std::uintptr_t>& o,
                                std::size_t query_heads, AttentionPrecision precision, std::size_t reps) {
        if (q.size() != seqs.size() || o.size() != seqs.size()) {
            throw std::invalid_argument("one query and one output buffer per sequence");
        }
        py::gil_scoped_release release;
        return seconds_per_call(reps, [&] {
            for (std::size_t i = 0; i < seqs.size(); ++i) {
                paged_attention(s, *seqs[i], static_cast<const float*>(ptr(q[i])), static_cast<float*>(ptr(o[i])),
                                seqs[i]->num_tokens(), query_heads, precision);
            }
        });
    }, "all sequences' tokens as queries (whole-prompt prefill), one call per sequence");
}

static void bind_v3(py::module_ v3m) {
    namespace v3 = kvflux::v3;
    py::enum_<v3::StorageTier>(v3m, "StorageTier")
        .value("GPU", v3::StorageTier::GPU)
        .value("CPU", v3::StorageTier::CPU)
        .value("NVME", v3::StorageTier::NVME);
    py::enum_<v3::ChunkState>(v3m, "ChunkState")
        .value("READY", v3::ChunkState::READY)
        .value("COPYING", v3::ChunkState::COPYING)
        .value("LOADING", v3::ChunkState::LOADING)
        .value("EVICTING", v3::ChunkState::EVICTING)
        .value("ERROR", v3::ChunkState::ERROR);
    py::class_<v3::TierLocation>(v3m, "TierLocation")
        .def(py::init([](std::size_t slot, std::uint64_t generation) { return v3::TierLocation{slot, generation}; }),
             py::arg("slot"), py::arg("generation"))
        .def_readonly("slot", &v3::TierLocation::slot)
        .def_readonly("generation", &v3::TierLocation::generation)
        .def("__eq__", &v3::TierLocation::operator==);
    py::class_<v3::Tier>(v3m, "Tier")
        .def("kind", &v3::Tier::kind)
        .def("chunk_bytes", &v3::Tier::chunk_bytes)
        .def("capacity", &v3::Tier::capacity)
        .def("allocated_chunks", &v3::Tier::allocated_chunks)
        .def("available", &v3::Tier::available)
        .def("used_bytes", &v3::Tier::used_bytes)
        .def("available_bytes", &v3::Tier::available_bytes)
        .def("allocate", &v3::Tier::allocate)
        .def("release", &v3::Tier::release);
    py::class_<v3::SlotTier, v3::Tier>(v3m, "SlotTier");
    py::class_<v3::CpuTier, v3::SlotTier>(v3m, "CpuTier").def(py::init<std::size_t, std::size_t>());
    py::class_<v3::NvmeTier, v3::SlotTier>(v3m, "NvmeTier").def(py::init<std::size_t, std::size_t>());
    py::class_<v3::GpuTier, v3::Tier>(v3m, "GpuTier")
        .def(py::init<PhysicalBlockPool&, std::size_t>(), py::keep_alive<1, 2>());
    py::class_<v3::CacheKey>(v3m, "CacheKey")
        .def_readonly("model_id", &v3::CacheKey::model_id)
        .def_readonly("prefix_hash", &v3::CacheKey::prefix_hash)
        .def_readonly("prefix", &v3::CacheKey::prefix)
        .def("__eq__", &v3::CacheKey::operator==);
    v3m.def("make_cache_key", &v3::make_cache_key);
    py::class_<v3::Replica>(v3m, "Replica")
        .def_readonly("location", &v3::Replica::location)
        .def_readonly("state", &v3::Replica::state);
    py::class_<v3::ChunkRecord>(v3m, "ChunkRecord")
        .def_readonly("version", &v3::ChunkRecord::version)
        .def_readonly("ref_count", &v3::ChunkRecord::ref_count)
        .def_readonly("pin_count", &v3::ChunkRecord::pin_count)
        .def_readonly("gpu", &v3::ChunkRecord::gpu)
        .def_readonly("cpu", &v3::ChunkRecord::cpu)
        .def_readonly("nvme", &v3::ChunkRecord::nvme);
    py::class_<v3::CacheDirectory>(v3m, "CacheDirectory")
        .def(py::init<v3::Tier&, v3::Tier&, v3::Tier&>(), py::keep_alive<1, 2>(), py::keep_alive<1, 3>(),
             py::keep_alive<1, 4>())
        .def("create", &v3::CacheDirectory::create)
        .def("contains", &v3::CacheDirectory::contains)
        .def("at", &v3::CacheDirectory::at, py::return_value_policy::copy)
        .def("size", &v3::CacheDirectory::size)
        .def("place", &v3::CacheDirectory::place, py::arg("key"), py::arg("tier"),
             py::arg("state") = v3::ChunkState::READY)
        .def("remove", &v3::CacheDirectory::remove)
        .def("set_state", &v3::CacheDirectory::set_state)
        .def("pin", &v3::CacheDirectory::pin)
        .def("unpin", &v3::CacheDirectory::unpin)
        .def("destroy", &v3::CacheDirectory::destroy)
        .def("replica_count", &v3::CacheDirectory::replica_count);
    py::class_<v3::HostChunkBuffers>(v3m, "HostChunkBuffers")
        .def("chunk_bytes", &v3::HostChunkBuffers::chunk_bytes)
        .def("slots", &v3::HostChunkBuffers::slots)
        .def("data", [](v3::HostChunkBuffers& b, std::size_t slot) { return addr(b.data(slot)); });
    py::class_<v3::HeapChunkPool, v3::HostChunkBuffers>(v3m, "HeapChunkPool")
        .def(py::init<std::size_t, std::size_t>());
    py::class_<v3::PinnedChunkPool, v3::HostChunkBuffers>(v3m, "PinnedChunkPool")
        .def(py::init<std::size_t, std::size_t>())
        .def("device_data", [](const v3::PinnedChunkPool& b, std::size_t slot) { return addr(b.device_data(slot)); });
    py::class_<v3::GpuChunkStore>(v3m, "GpuChunkStore")
        .def(py::init<std::size_t, std::size_t, int>(), py::arg("total_slots"), py::arg("chunk_bytes"),
             py::arg("device") = 0)
        .def("device_ptr", [](const v3::GpuChunkStore& g, const v3::TierLocation& l) { return addr(g.device_ptr(l)); })
        .def("chunk_bytes", &v3::GpuChunkStore::chunk_bytes)
        .def("slots", &v3::GpuChunkStore::slots);
    py::class_<v3::GpuCpuTransfer>(v3m, "GpuCpuTransfer")
        .def(py::init<v3::CacheDirectory&, v3::GpuChunkStore&, v3::HostChunkBuffers&, int>(), py::arg("directory"),
             py::arg("gpu_store"), py::arg("cpu_buffers"), py::arg("device") = 0, py::keep_alive<1, 2>(),
             py::keep_alive<1, 3>(), py::keep_alive<1, 4>())
        .def("begin_offload", [](v3::GpuCpuTransfer& t, const v3::CacheKey& k) { t.begin_offload(k); })
        .def("begin_onload", [](v3::GpuCpuTransfer& t, const v3::CacheKey& k) { t.begin_onload(k); })
        .def("begin_offload_batch", [](v3::GpuCpuTransfer& t, const std::vector<v3::CacheKey>& k) {
            t.begin_offload(k);
        })
        .def("begin_onload_batch", [](v3::GpuCpuTransfer& t, const std::vector<v3::CacheKey>& k) {
            t.begin_onload(k);
        })
        .def("finish_offload", [](v3::GpuCpuTransfer& t, const v3::CacheKey& k, bool release) {
            py::gil_scoped_release unlock;
            t.finish_offload(k, release);
        })
        .def("finish_onload", [](v3::GpuCpuTransfer& t, const v3::CacheKey& k, bool release) {
            py::gil_scoped_release unlock;
            t.finish_onload(k, release);
        })
        .def("has_pending", &v3::GpuCpuTransfer::has_pending)
        .def("stream", [](const v3::GpuCpuTransfer& t) { return addr(t.stream()); });
}

PYBIND11_MODULE(_kvflux, m) {
    m.doc() = "kvflux::v2 paged-KV data path (MI355X / gfx950)";

    static py::exception<CapacityError> capacity_error(m, "CapacityError", PyExc_RuntimeError);
    static py::exception<std::logic_error> logic_error(m, "LogicError", PyExc_RuntimeError);
    py::register_exception_translator([](std::exception_ptr p) {
        try {
            if (p) std::rethrow_exception(p);
        } catch (const CapacityError& e) {
            py::set_error(capacity_error, e.what());
        } catch (const std::invalid_argument& e) {
            py::set_error(PyExc_ValueError, e.what());
        } catch (const std::out_of_range& e) {
            py::set_error(PyExc_IndexError, e.what());
        } catch (const std::logic_error& e) {
            py::set_error(logic_error, e.what());
        }
    });

    py::enum_<DType>(m, "DType")
        .value("Float16", DType::Float16)
        .value("BFloat16", DType::BFloat16)
        .value("Float32", DType::Float32);
    py::enum_<KVKind>(m, "KVKind").value("Key", KVKind::Key).value("Value", KVKind::Value);
    py::enum_<AttentionPrecision>(m, "AttentionPrecision")
        .value("Exact", AttentionPrecision::Exact)
        .value("Auto", AttentionPrecision::Auto)
        .value("Fast", AttentionPrecision::Fast);

    py::class_<BlockHandle>(m, "PhysicalBlockHandle")
        .def(py::init([](std::size_t id, std::uint64_t generation) {
                 return BlockHandle{id, generation};
             }),
             py::arg("id"), py::arg("generation"))
        .def_readonly("id", &BlockHandle::id)
        .def_readonly("generation", &BlockHandle::generation)
        .def("__eq__", [](const BlockHandle& a, const BlockHandle& b) { return a == b; })
        .def("__hash__", [](const BlockHandle& h) { return py::hash(py::make_tuple(h.id, h.generation)); })
        .def("__repr__", [](const BlockHandle& h) {
            return "PhysicalBlockHandle(" + std::to_string(h.id) + ", " + std::to_string(h.generation) + ")";
        });

    py::class_<PhysicalBlockPool>(m, "PhysicalBlockPool")
        .def(py::init([](std::size_t capacity, std::size_t block_size, py::object hasher) {
                 if (hasher.is_none()) return new PhysicalBlockPool(capacity, block_size);
                 auto fn = hasher.cast<std::function<std::uint64_t(const Tokens&)>>();
                 return new PhysicalBlockPool(capacity, block_size, fn);
             }),
             py::arg("capacity"), py::arg("block_size"), py::arg("hasher") = py::none())
        .def("allocate", &PhysicalBlockPool::allocate)
        .def("retain", &PhysicalBlockPool::retain)
        .def("free", &PhysicalBlockPool::free)
        .def("publish", &PhysicalBlockPool::publish)
        .def("lookup", [](PhysicalBlockPool& pool, const Tokens& prefix) -> py::object {
            PhysicalBlockHandle out{};
            if (!pool.lookup(prefix, out)) return py::none();
            return py::cast(out);
        })
        .def("is_published", &PhysicalBlockPool::is_published)
        .def("id", &PhysicalBlockPool::id)
        .def("ref_count", &PhysicalBlockPool::ref_count)
        .def("capacity", &PhysicalBlockPool::capacity)
        .def("block_size", &PhysicalBlockPool::block_size)
        .def("available", &PhysicalBlockPool::available);

    m.def("prefix_hash", &BlockManager::prefix_hash);

    py::class_<BlockTable>(m, "BlockTable")
        .def(py::init<PhysicalBlockPool&>(), py::keep_alive<1, 2>())
        .def("append_new", &BlockTable::append_new)
        .def("append_existing", &BlockTable::append_existing)
        .def("append_shared", &BlockTable::append_shared)
        .def("physical_id", &BlockTable::physical_id)
        .def("handle", &BlockTable::handle)
        .def("ref_count", &BlockTable::ref_count)
        .def("__getitem__", &BlockTable::operator[])
        .def("__len__", &BlockTable::size)
        .def("size", &BlockTable::size)
        .def("empty", &BlockTable::empty)
        .def("shares_pool_with", &BlockTable::shares_pool_with)
        .def("uses_pool", &BlockTable::uses_pool)
        .def("pop_back", &BlockTable::pop_back)
        .def("replace_last_owned", &BlockTable::replace_last_owned)
        .def("clear", &BlockTable::clear)
        .def("move_from", [](BlockTable& self, BlockTable& other) { self = std::move(other); },
             "C++ move assignment: self = std::move(other)")
        .def_static("moved", [](BlockTable& other) { return BlockTable(std::move(other)); },
                    "C++ move construction from `other`");

    py::class_<TokenLocation>(m, "TokenLocation")
        .def_readonly("physical_block", &TokenLocation::physical_block)
        .def_readonly("offset_in_block", &TokenLocation::offset_in_block);

    py::class_<SequenceState>(m, "SequenceState")
        .def(py::init<RequestID, PhysicalBlockPool&>(), py::keep_alive<1, 3>())
        .def("request_id", &SequenceState::request_id)
        .def("num_tokens", &SequenceState::num_tokens)
        .def("block_size", &SequenceState::block_size)
        .def("block_table", &SequenceState::block_table, py::return_value_policy::reference_internal)
        .def("num_allocated_blocks", &SequenceState::num_allocated_blocks)
        .def("last_block_num_tokens", &SequenceState::last_block_num_tokens)
        .def("append_tokens", &SequenceState::append_tokens)
        .def("append_token", &SequenceState::append_token)
        .def("fork_shared", [](const SequenceState& s, RequestID id) {
            // The fork must keep the pool alive, not the source sequence.
            py::object fork = py::cast(s.fork_shared(id));
            py::object pool = py::cast(&s.block_table().pool(), py::return_value_policy::reference);
            py::detail::keep_alive_impl(fork, pool);
            return fork;
        })
        .def("append_token_with_copy", &SequenceState::append_token_with_copy)
        .def("physical_block_id", &SequenceState::physical_block_id)
        .def("token_location", &SequenceState::token_location)
        .def("move_from", [](SequenceState& self, SequenceState& other) { self = std::move(other); },
             "C++ move assignment: self = std::move(other)");

    m.def("build_slot_mapping", [](const std::vector<std::pair<const SequenceState*, std::size_t>>& batch) {
        std::vector<TokenWrite> writes;
        writes.reserve(batch.size());
        for (const auto& [seq, pos] : batch) writes.push_back({seq, pos});
        return build_slot_mapping(writes);
    }, py::arg("batch"), "batch: list of (SequenceState or None, token_position)");

    py::class_<BatchBlockTable>(m, "BatchBlockTable")
        .def("num_sequences", &BatchBlockTable::num_sequences)
        .def("max_blocks_per_sequence", &BatchBlockTable::max_blocks_per_sequence)
        .def("block_table", &BatchBlockTable::block_table)
        .def("sequence_lengths", &BatchBlockTable::sequence_lengths)
        .def_static("invalid_block", &BatchBlockTable::invalid_block)
        .def("physical_id", &BatchBlockTable::physical_id);
    m.def("build_batch_block_table", &build_batch_block_table);

    py::class_<PrefixCache>(m, "PrefixCache")
        .def(py::init<PhysicalBlockPool&>(), py::keep_alive<1, 2>())
        .def("attach_cached_prefix", &PrefixCache::attach_cached_prefix)
        .def("publish_computed_block", &PrefixCache::publish_computed_block);
    m.def("build_read_block_table", &build_read_block_table);

    py::class_<PagedKVLayout>(m, "PagedKVLayout")
        .def(py::init<std::size_t, std::size_t, std::size_t, std::size_t, DType>())
        .def("num_blocks", &PagedKVLayout::num_blocks)
        .def("num_kv_heads", &PagedKVLayout::num_kv_heads)
        .def("block_size", &PagedKVLayout::block_size)
        .def("head_size", &PagedKVLayout::head_size)
        .def("dtype", &PagedKVLayout::dtype)
        .def("element_bytes", &PagedKVLayout::element_bytes)
        .def("page_bytes", &PagedKVLayout::page_bytes)
        .def("cache_bytes", &PagedKVLayout::cache_bytes)
        .def("total_bytes", &PagedKVLayout::total_bytes)
        .def("slot_count", &PagedKVLayout::slot_count)
        .def("page_byte_offset", &PagedKVLayout::page_byte_offset)
        .def("byte_offset", &PagedKVLayout::byte_offset)
        .def("slot_byte_offset", &PagedKVLayout::slot_byte_offset);

    py::class_<PagedKVStorage>(m, "PagedKVStorage")
        .def(py::init<PhysicalBlockPool&, std::size_t, std::size_t, DType, int>(),
             py::arg("pool"), py::arg("num_kv_heads"), py::arg("head_size"), py::arg("dtype"),
             py::arg("device") = 0, py::keep_alive<1, 2>())
        .def("layout", &PagedKVStorage::layout, py::return_value_policy::reference_internal)
        .def("device", &PagedKVStorage::device)
        .def("uses_pool", &PagedKVStorage::uses_pool)
        .def("key_base", [](const PagedKVStorage& s) { return addr(s.key_base()); })
        .def("value_base", [](const PagedKVStorage& s) { return addr(s.value_base()); })
        .def("page_address", [](const PagedKVStorage& s, KVKind k, PhysicalBlockHandle h) {
            return addr(s.page_address(k, h));
        })
        .def("element_address", [](const PagedKVStorage& s, KVKind k, PhysicalBlockHandle h,
                                   std::size_t head, std::size_t token, std::size_t dim) {
            return addr(s.element_address(k, h, head, token, dim));
        })
        .def("slot_address", [](const PagedKVStorage& s, KVKind k, PhysicalSlot slot,
                                std::size_t head, std::size_t dim) {
            return addr(s.slot_address(k, slot, head, dim));
        })
        .def("copy_block", &PagedKVStorage::copy_block)
        .def("copy_blocks", [](const PagedKVStorage& s,
                               const std::vector<std::pair<PhysicalBlockHandle, PhysicalBlockHandle>>& pairs) {
            py::gil_scoped_release release;
            s.copy_blocks(pairs);
        });

    m.def("append_token_cow", &append_token_cow);
    m.def("append_tokens_cow", [](const PagedKVStorage& s, const std::vector<SequenceState*>& seqs) {
        py::gil_scoped_release release;
        return append_tokens_cow(s, seqs);
    });

    py::class_<DeviceBatchTable>(m, "DeviceBatchTable")
        .def(py::init<const PagedKVStorage&, std::vector<SequenceState*>, std::size_t>(),
             py::arg("storage"), py::arg("sequences"), py::arg("capacity_blocks"),
             py::keep_alive<1, 2>(), py::keep_alive<1, 3>())
        .def("refresh", [](DeviceBatchTable& t) {
            py::gil_scoped_release release;
            t.refresh();
        })
        .def("rows", &DeviceBatchTable::rows)
        .def("capacity_blocks", &DeviceBatchTable::capacity_blocks)
        .def("lengths", &DeviceBatchTable::lengths)
        .def("device_table", [](const DeviceBatchTable& t) { return addr(t.device_table()); })
        .def("device_lengths", [](const DeviceBatchTable& t) { return addr(t.device_lengths()); });
    m.def("decode_step", [](PagedKVStorage& s, DeviceBatchTable& t, std::uintptr_t k, std::uintptr_t v,
                            std::uintptr_t q, std::uintptr_t o, std::size_t query_heads) {
        py::gil_scoped_release release;
        return decode_step(s, t, ptr(k), ptr(v), static_cast<const float*>(ptr(q)),
                           static_cast<float*>(ptr(o)), query_heads);
    });

    py::class_<SequenceLifecycle>(m, "SequenceLifecycle")
        .def(py::init<RequestID, PhysicalBlockPool&, PagedKVStorage&, std::size_t, AttentionPrecision>(),
             py::arg("request_id"), py::arg("pool"), py::arg("storage"), py::arg("query_heads"),
             py::arg("precision") = AttentionPrecision::Exact, py::keep_alive<1, 3>(), py::keep_alive<1, 4>())
        .def("prefill", [](SequenceLifecycle& s, std::size_t n, std::uintptr_t k, std::uintptr_t v,
                           std::uintptr_t q, std::uintptr_t o) {
            py::gil_scoped_release release;
            s.prefill(n, ptr(k), ptr(v), static_cast<const float*>(ptr(q)), static_cast<float*>(ptr(o)));
        })
        .def("decode", [](SequenceLifecycle& s, std::uintptr_t k, std::uintptr_t v, std::uintptr_t q,
                          std::uintptr_t o) {
            py::gil_scoped_release release;
            return s.decode(ptr(k), ptr(v), static_cast<const float*>(ptr(q)), static_cast<float*>(ptr(o)));
        })
        .def("finish", &SequenceLifecycle::finish)
        .def("finished", &SequenceLifecycle::finished)
        .def("sequence", &SequenceLifecycle::sequence, py::return_value_policy::reference_internal);

    m.def("write_paged_kv", [](PagedKVStorage& s, std::uintptr_t k, std::uintptr_t v,
                               const SlotMapping& slots) {
        py::gil_scoped_release release;
        write_paged_kv(s, ptr(k), ptr(v), slots);
    });
    m.def("read_paged_kv", [](const PagedKVStorage& s, const SequenceState& seq, std::uintptr_t k,
                              std::uintptr_t v) {
        py::gil_scoped_release release;
        read_paged_kv(s, seq, ptr(k), ptr(v));
    });
    m.def("read_paged_kv_batch", [](const PagedKVStorage& s,
                                    const std::vector<const SequenceState*>& seqs,
                                    std::uintptr_t k, std::uintptr_t v) {
        py::gil_scoped_release release;
        read_paged_kv_batch(s, seqs, ptr(k), ptr(v));
    });
    m.def("paged_attention", [](const PagedKVStorage& s, const SequenceState& seq,
                                std::uintptr_t q, std::uintptr_t o, std::size_t query_tokens,
                                std::size_t query_heads, AttentionPrecision precision) {
        py::gil_scoped_release release;
        paged_attention(s, seq, static_cast<const float*>(ptr(q)), static_cast<float*>(ptr(o)),
                        query_tokens, query_heads, precision);
    }, py::arg("storage"), py::arg("sequence"), py::arg("query"), py::arg("output"),
       py::arg("query_tokens"), py::arg("query_heads"),
       py::arg("precision") = AttentionPrecision::Exact);
    py::class_<AttentionShape>(m, "AttentionShape")
        .def(py::init([](std::size_t qt, std::size_t kt, std::size_t qh, std::size_t kh, std::size_t d) {
                 return AttentionShape{qt, kt, qh, kh, d};
             }),
             py::arg("query_tokens"), py::arg("kv_tokens"), py::arg("query_heads"), py::arg("kv_heads"),
             py::arg("head_size"))
        .def_readwrite("query_tokens", &AttentionShape::query_tokens)
        .def_readwrite("kv_tokens", &AttentionShape::kv_tokens)
        .def_readwrite("query_heads", &AttentionShape::query_heads)
        .def_readwrite("kv_heads", &AttentionShape::kv_heads)
        .def_readwrite("head_size", &AttentionShape::head_size);
    m.def("reference_attention", &reference_attention, py::arg("query"), py::arg("key"), py::arg("value"),
          py::arg("shape"));
    m.def("paged_attention_batch", [](const PagedKVStorage& s,
                                      const std::vector<const SequenceState*>& seqs,
                                      std::uintptr_t q, std::uintptr_t o, std::size_t query_heads) {
        py::gil_scoped_release release;
        paged_attention_batch(s, seqs, static_cast<const float*>(ptr(q)),
                              static_cast<float*>(ptr(o)), query_heads);
    });
    bind_v3(m.def_submodule("v3", "kvflux::v3 tiered cache: tiers, directory, GPU <-> CPU transfer"));
    bind_timing(m.def_submodule("timing", "seconds per call of the synchronous C++ API, timed in C++"));
    m.def("paged_attention_batch", [](const PagedKVStorage& s, const DeviceBatchTable& t,
                                      std::uintptr_t q, std::uintptr_t o, std::size_t query_heads) {
        py::gil_scoped_release release;
        paged_attention_batch(s, t, static_cast<const float*>(ptr(q)), static_cast<float*>(ptr(o)),
                              query_heads);
    });
}
