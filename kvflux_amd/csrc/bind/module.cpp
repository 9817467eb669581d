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
        .def(py::init<RequestID, PhysicalBlockPool&, PagedKVStorage&, std::size_t>(),
             py::keep_alive<1, 3>(), py::keep_alive<1, 4>())
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
       py::arg("precision") = AttentionPrecision::Auto);
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
    m.def("paged_attention_batch", [](const PagedKVStorage& s, const DeviceBatchTable& t,
                                      std::uintptr_t q, std::uintptr_t o, std::size_t query_heads) {
        py::gil_scoped_release release;
        paged_attention_batch(s, t, static_cast<const float*>(ptr(q)), static_cast<float*>(ptr(o)),
                              query_heads);
    });
}
