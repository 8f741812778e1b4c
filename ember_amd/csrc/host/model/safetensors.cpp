// Parsing safetensors headers over mapped files, with every byte range checked
// against its file and its dtype x shape.
#include "model/safetensors.hpp"

#include <cstring>
#include <set>

#include "common/error.hpp"
#include "common/json.hpp"

namespace ember {

const char *dtype_name(DType t) {
    switch (t) {
        case DType::f32: return "F32";
        case DType::f16: return "F16";
        case DType::bf16: return "BF16";
        case DType::i8: return "I8";
        case DType::u8: return "U8";
        case DType::i32: return "I32";
        case DType::i64: return "I64";
    }
    return "?";
}

size_t dtype_size(DType t) {
    switch (t) {
        case DType::f32: case DType::i32: return 4;
        case DType::f16: case DType::bf16: return 2;
        case DType::i8: case DType::u8: return 1;
        case DType::i64: return 8;
    }
    return 0;
}

namespace {

DType parse_dtype(const std::string &s, const std::string &tensor) {
    static const std::pair<const char *, DType> names[] = {{"F32", DType::f32}, {"F16", DType::f16},
                                                           {"BF16", DType::bf16}, {"I8", DType::i8},
                                                           {"U8", DType::u8}, {"I32", DType::i32},
                                                           {"I64", DType::i64}};
    for (const auto &[n, t] : names)
        if (s == n) return t;
    fail("tensor {}: unsupported dtype {}", tensor, s);
}

}  // namespace

std::string TensorView::shape_str() const {
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); i++) s += (i ? ", " : "") + std::to_string(shape[i]);
    return s + "]";
}

void SafeTensors::add_file(const std::string &path) {
    auto file = std::make_unique<MappedFile>(path);
    const uint8_t *base = file->data();
    const size_t size = file->size();
    EMBER_CHECK(size >= 8, "{}: too short for a safetensors file", path);
    uint64_t header_len = 0;
    for (int i = 7; i >= 0; i--) header_len = (header_len << 8) | base[i];  // little-endian
    EMBER_CHECK(header_len <= size - 8, "{}: header length {} past the end of the file", path, header_len);
    const json::Value header =
        json::Value::parse(std::string_view(reinterpret_cast<const char *>(base + 8), static_cast<size_t>(header_len)));
    const uint8_t *data = base + 8 + header_len;
    const size_t data_size = size - 8 - static_cast<size_t>(header_len);
    for (const auto &[name, desc] : header.as_object()) {
        if (name == "__metadata__") continue;
        EMBER_CHECK(!tensors_.count(name), "tensor {} appears twice", name);
        TensorView t;
        t.name = name;
        t.dtype = parse_dtype(desc["dtype"].as_string(), name);
        for (const json::Value &d : desc["shape"].as_array()) {
            t.shape.push_back(d.as_int());
            EMBER_CHECK(t.shape.back() >= 0, "tensor {}: negative dimension", name);
        }
        const json::Value &off = desc["data_offsets"];
        EMBER_CHECK(off.size() == 2, "tensor {}: data_offsets needs two entries", name);
        const int64_t begin = off[0].as_int(), end = off[1].as_int();
        EMBER_CHECK(0 <= begin && begin <= end && static_cast<uint64_t>(end) <= data_size,
                    "tensor {}: byte range [{}, {}) outside the data ({} bytes)", name, begin, end, data_size);
        t.bytes = static_cast<size_t>(end - begin);
        EMBER_CHECK(t.bytes == static_cast<size_t>(t.numel()) * dtype_size(t.dtype),
                    "tensor {}: {} bytes for {} x {}", name, t.bytes, t.shape_str(), dtype_name(t.dtype));
        t.data = data + begin;
        tensors_.emplace(name, std::move(t));
    }
    files_.push_back(std::move(file));
}

SafeTensors SafeTensors::open_file(const std::string &path) {
    SafeTensors st;
    st.add_file(path);
    return st;
}

SafeTensors SafeTensors::open_dir(const std::string &dir) {
    SafeTensors st;
    const std::string index = dir + "/model.safetensors.index.json";
    if (file_exists(index)) {
        const json::Value idx = json::Value::parse(read_file(index));
        std::set<std::string> shards;
        for (const auto &[name, file] : idx["weight_map"].as_object()) shards.insert(file.as_string());
        for (const std::string &f : shards) {
            EMBER_CHECK(f.find('/') == std::string::npos, "shard name {} leaves the model directory", f);
            st.add_file(dir + "/" + f);
        }
        return st;
    }
    st.add_file(dir + "/model.safetensors");
    return st;
}

const TensorView &SafeTensors::get(const std::string &name) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) fail("tensor {} is missing from the model", name);
    return it->second;
}

const TensorView &SafeTensors::get(const std::string &name, const std::vector<int64_t> &shape) const {
    const TensorView &t = get(name);
    if (t.shape != shape) {
        TensorView want;
        want.shape = shape;
        fail("tensor {} has shape {}, expected {}", name, t.shape_str(), want.shape_str());
    }
    return t;
}

size_t SafeTensors::total_bytes() const {
    size_t n = 0;
    for (const auto &[name, t] : tensors_) n += t.bytes;
    return n;
}

}  // namespace ember
