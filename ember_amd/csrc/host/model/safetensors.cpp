// Reading safetensors files over memory maps. The format: bytes 0..7 hold N,
// the header's length (unsigned 64-bit, little-endian); bytes 8..8+N hold a
// JSON object mapping each tensor name to {"dtype", "shape", "data_offsets":
// [begin, end]} (offsets relative to the byte after the header), plus an
// optional "__metadata__" entry; the tensor bytes follow. A sharded model adds
// model.safetensors.index.json, whose "weight_map" names each tensor's file.
// Every byte range is checked against its file and against dtype x shape.
#include "model/safetensors.hpp"

#include <algorithm>
#include <cstring>

#include "common/error.hpp"
#include "common/json.hpp"

namespace ember {

namespace {

struct DTypeInfo {
    DType type;
    const char *name;  // the header's spelling
    size_t bytes;
};

constexpr DTypeInfo kDTypes[] = {
    {DType::f32, "F32", 4}, {DType::f16, "F16", 2}, {DType::bf16, "BF16", 2}, {DType::i8, "I8", 1},
    {DType::u8, "U8", 1},   {DType::i32, "I32", 4}, {DType::i64, "I64", 8},
};

const DTypeInfo *info_of(DType t) {
    const auto hit = std::find_if(std::begin(kDTypes), std::end(kDTypes), [t](const DTypeInfo &d) { return d.type == t; });
    return hit == std::end(kDTypes) ? nullptr : hit;
}

// Reads one header entry into a view of the data section [data, data + data_bytes).
TensorView read_entry(const std::string &file, const std::string &name, const json::Value &entry, const uint8_t *data,
                      uint64_t data_bytes) {
    TensorView t;
    t.name = name;
    const std::string &dtype = entry["dtype"].as_string();
    const auto kind = std::find_if(std::begin(kDTypes), std::end(kDTypes),
                                   [&dtype](const DTypeInfo &d) { return dtype == d.name; });
    if (kind == std::end(kDTypes)) fail("{}: tensor {} has dtype {}, which is not supported", file, name, dtype);
    t.dtype = kind->type;

    const json::Value &shape = entry["shape"];
    t.shape.reserve(shape.size());
    for (size_t i = 0; i < shape.size(); ++i) {
        const int64_t extent = shape[i].as_int();
        if (extent < 0) fail("{}: tensor {} has a negative extent in its shape", file, name);
        t.shape.push_back(extent);
    }

    const json::Value &range = entry["data_offsets"];
    if (range.size() != 2) fail("{}: tensor {} needs data_offsets [begin, end]", file, name);
    const int64_t begin = range[0].as_int(), end = range[1].as_int();
    if (begin < 0 || end < begin || static_cast<uint64_t>(end) > data_bytes)
        fail("{}: tensor {} spans bytes [{}, {}) of a {}-byte data section", file, name, begin, end, data_bytes);
    t.bytes = static_cast<size_t>(end - begin);
    const uint64_t expected = static_cast<uint64_t>(t.numel()) * kind->bytes;
    if (t.bytes != expected)
        fail("{}: tensor {} holds {} bytes, but {} of {} need {}", file, name, t.bytes, t.shape_str(), dtype, expected);
    t.data = data + begin;
    return t;
}

}  // namespace

const char *dtype_name(DType t) {
    const DTypeInfo *d = info_of(t);
    return d != nullptr ? d->name : "?";
}

size_t dtype_size(DType t) {
    const DTypeInfo *d = info_of(t);
    return d != nullptr ? d->bytes : 0;
}

std::string TensorView::shape_str() const {
    std::string s(1, '[');
    for (size_t i = 0; i < shape.size(); ++i) {
        if (i > 0) s += ", ";
        s += std::to_string(shape[i]);
    }
    s += ']';
    return s;
}

void SafeTensors::add_file(const std::string &path) {
    auto mapped = std::make_unique<MappedFile>(path);
    const uint64_t file_bytes = mapped->size();
    if (file_bytes < 8) fail("{}: {} bytes, shorter than a safetensors length prefix", path, file_bytes);
    uint8_t prefix[8];
    std::memcpy(prefix, mapped->data(), 8);
    uint64_t header_bytes = 0;
    for (int b = 0; b < 8; ++b) header_bytes |= static_cast<uint64_t>(prefix[b]) << (8 * b);
    if (header_bytes > file_bytes - 8)
        fail("{}: the header claims {} bytes, past the end of the file ({} bytes)", path, header_bytes, file_bytes);

    const char *header_text = reinterpret_cast<const char *>(mapped->data() + 8);
    const json::Value header = json::Value::parse(std::string_view(header_text, static_cast<size_t>(header_bytes)));
    const uint8_t *data = mapped->data() + 8 + header_bytes;
    const uint64_t data_bytes = file_bytes - 8 - header_bytes;

    for (const auto &member : header.as_object()) {
        const std::string &name = member.first;
        if (name == "__metadata__") continue;
        if (tensors_.find(name) != tensors_.end()) fail("{}: tensor {} is already defined by another file", path, name);
        tensors_.emplace(name, read_entry(path, name, member.second, data, data_bytes));
    }
    files_.push_back(std::move(mapped));
}

SafeTensors SafeTensors::open_file(const std::string &path) {
    SafeTensors st;
    st.add_file(path);
    return st;
}

SafeTensors SafeTensors::open_dir(const std::string &dir) {
    SafeTensors st;
    const std::string index_path = dir + "/model.safetensors.index.json";
    if (!file_exists(index_path)) {
        st.add_file(dir + "/model.safetensors");
        return st;
    }
    // The index maps tensor -> shard file; each shard is opened once, in name order.
    const json::Value index = json::Value::parse(read_file(index_path));
    std::vector<std::string> shards;
    for (const auto &entry : index["weight_map"].as_object()) shards.push_back(entry.second.as_string());
    std::sort(shards.begin(), shards.end());
    shards.erase(std::unique(shards.begin(), shards.end()), shards.end());
    for (const std::string &shard : shards) {
        if (shard.empty() || shard.find('/') != std::string::npos || shard == "..")
            fail("{}: shard name \"{}\" is not a file in the model directory", index_path, shard);
        st.add_file(dir + "/" + shard);
    }
    return st;
}

const TensorView &SafeTensors::get(const std::string &name) const {
    const auto it = tensors_.find(name);
    if (it == tensors_.end()) fail("the model has no tensor {}", name);
    return it->second;
}

const TensorView &SafeTensors::get(const std::string &name, const std::vector<int64_t> &shape) const {
    const TensorView &t = get(name);
    if (t.shape == shape) return t;
    TensorView wanted;
    wanted.shape = shape;
    fail("tensor {} has shape {}, but {} is required", name, t.shape_str(), wanted.shape_str());
}

size_t SafeTensors::total_bytes() const {
    size_t sum = 0;
    for (const auto &entry : tensors_) sum += entry.second.bytes;
    return sum;
}

}  // namespace ember
