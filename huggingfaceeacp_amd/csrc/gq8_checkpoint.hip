// gq8_checkpoint.hip -- safetensors files and Gemma's config.json on the
// host, and their C ABI (include/gemma_q8.h).  The rules follow the
// reference's loader: Model/SafeTensors.cpp (header checks, widening),
// Model/TensorType.h (dtype tags), Model/GemmaConfig.cpp (config fields).
#include "gemma_q8.h"
#include "gq8_checkpoint.hpp"
#include "gq8_json.hpp"
#include "gq8_numerics.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstring>
#include <limits>
#include <memory>
#include <utility>

namespace gq8 {
namespace {

const char *const kDtypeNames[kDtypeCount] = {"BOOL", "U8", "I8", "U16", "I16", "F16", "BF16",
                                              "U32", "I32", "F32", "U64", "I64", "F64"};
const int kDtypeBytes[kDtypeCount] = {1, 1, 1, 2, 2, 2, 2, 4, 4, 4, 8, 8, 8};

int dtype_of(const std::string &name)
{
    for (int i = 0; i < kDtypeCount; ++i)
        if (name == kDtypeNames[i])
            return i;
    return -1;
}

int format_error(const std::string &message)
{
    return report(GQ8_ERR_FORMAT, message);
}

} // namespace

int dtype_bytes(int dtype)
{
    return dtype >= 0 && dtype < kDtypeCount ? kDtypeBytes[dtype] : 0;
}

const char *dtype_name(int dtype)
{
    return dtype >= 0 && dtype < kDtypeCount ? kDtypeNames[dtype] : "";
}

int64_t TensorInfo::elements() const
{
    int64_t n = 1;
    for (int64_t d : shape)
        n *= d;
    return n;
}

SafeTensorsFile::~SafeTensorsFile()
{
    if (mapping_)
        (void) munmap(mapping_, size_);
}

int SafeTensorsFile::open(const std::string &path, SafeTensorsFile **out)
{
    *out = nullptr;
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0)
        return format_error("cannot open " + path);
    struct stat st {};
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        ::close(fd);
        return format_error(path + " is not a regular file");
    }
    std::unique_ptr<SafeTensorsFile> f(new SafeTensorsFile());
    f->size_ = (uint64_t) st.st_size;
    if (f->size_ > 0) {
        void *m = mmap(nullptr, f->size_, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            ::close(fd);
            return format_error("cannot map " + path);
        }
        f->mapping_ = m;
        f->data_ = static_cast<const uint8_t *>(m);
    }
    ::close(fd); // the mapping holds the file
    if (int s = f->parse_header())
        return s;
    *out = f.release();
    return GQ8_OK;
}

int SafeTensorsFile::from_bytes(const uint8_t *bytes, uint64_t size, SafeTensorsFile **out)
{
    *out = nullptr;
    std::unique_ptr<SafeTensorsFile> f(new SafeTensorsFile());
    f->owned_.assign(bytes, bytes + size);
    f->data_ = f->owned_.data();
    f->size_ = size;
    if (int s = f->parse_header())
        return s;
    *out = f.release();
    return GQ8_OK;
}

// SafeTensors.cpp's header rules: a length prefix inside the file, an object,
// dtype / shape / data_offsets on every tensor, a known dtype, non-negative
// dims, an ordered byte range inside the blob that the shape fills exactly,
// string-to-string metadata.
int SafeTensorsFile::parse_header()
{
    if (size_ < 8)
        return format_error("a safetensors file starts with an 8-byte header length");
    uint64_t length = 0;
    std::memcpy(&length, data_, 8);
    if (length > size_ - 8)
        return format_error("the header length runs past the end of the file");
    blob_ = 8 + length;
    const uint64_t blobSize = size_ - blob_;
    Json root;
    JsonReader reader(reinterpret_cast<const char *>(data_ + 8), (size_t) length);
    if (!reader.read(root))
        return format_error("the header is not valid JSON");
    if (root.kind != Json::Object)
        return format_error("the header is not a JSON object");
    for (const auto &m : root.members) {
        if (m.first == "__metadata__") {
            if (m.second.kind != Json::Object)
                return format_error("__metadata__ is not an object");
            for (const auto &kv : m.second.members) {
                if (kv.second.kind != Json::String)
                    return format_error("__metadata__ value '" + kv.first + "' is not a string");
                metadata_[kv.first] = kv.second.text;
            }
            continue;
        }
        const Json &e = m.second;
        if (e.kind != Json::Object)
            return format_error("tensor '" + m.first + "' is not an object");
        const Json *dtype = e.find("dtype"), *shape = e.find("shape"), *range = e.find("data_offsets");
        if (!dtype || !shape || !range)
            return format_error("tensor '" + m.first + "' lacks dtype, shape or data_offsets");
        if (dtype->kind != Json::String || dtype_of(dtype->text) < 0)
            return format_error("tensor '" + m.first + "' has an unknown dtype");
        if (shape->kind != Json::Array || range->kind != Json::Array || range->items.size() != 2)
            return format_error("tensor '" + m.first + "' has a malformed shape or byte range");
        TensorInfo t;
        t.name = m.first;
        t.dtype = dtype_of(dtype->text);
        uint64_t count = 1;
        bool overflow = false;
        for (const Json &d : shape->items) {
            if (d.kind != Json::Number || !d.integral || d.integer < 0)
                return format_error("tensor '" + m.first + "' has a negative or non-integer dimension");
            t.shape.push_back(d.integer);
            if (d.integer != 0 && count > std::numeric_limits<uint64_t>::max() / (uint64_t) d.integer)
                overflow = true;
            count *= (uint64_t) d.integer;
        }
        const Json &b0 = range->items[0], &b1 = range->items[1];
        if (b0.kind != Json::Number || b1.kind != Json::Number || !b0.integral || !b1.integral
            || b0.integer < 0 || b1.integer < b0.integer)
            return format_error("tensor '" + m.first + "' has a negative or reversed byte range");
        if ((uint64_t) b1.integer > blobSize)
            return format_error("tensor '" + m.first + "' runs past the end of the blob");
        t.offset = (uint64_t) b0.integer;
        t.bytes = (uint64_t) (b1.integer - b0.integer);
        if (overflow || count > std::numeric_limits<uint64_t>::max() / (uint64_t) dtype_bytes(t.dtype)
            || count * (uint64_t) dtype_bytes(t.dtype) != t.bytes)
            return format_error("tensor '" + m.first + "' has a shape that disagrees with its byte range");
        tensors_.push_back(std::move(t));
    }
    std::sort(tensors_.begin(), tensors_.end(),
              [](const TensorInfo &a, const TensorInfo &b) { return a.name < b.name; });
    return GQ8_OK;
}

int SafeTensorsFile::find(const std::string &name) const
{
    const auto it = std::lower_bound(tensors_.begin(), tensors_.end(), name,
                                     [](const TensorInfo &t, const std::string &n) { return t.name < n; });
    return it != tensors_.end() && it->name == name ? (int) (it - tensors_.begin()) : -1;
}

// widenTensorElements (SafeTensors.h:71-76): F32 as it lies, F16 through the
// IEEE half widening, BF16 as the top 16 bits of a float; every widening is
// exact.  F64 rounds to nearest, as a float conversion does.
int SafeTensorsFile::read_floats(const TensorInfo &t, int64_t first, int64_t count, float *out) const
{
    const int64_t n = t.elements();
    if (first < 0 || count < 0 || first > n || count > n - first)
        return report(GQ8_ERR_ARGUMENT, "read_floats: range outside tensor '" + t.name + "'");
    const uint8_t *src = blob_bytes(t);
    switch (t.dtype) {
    case kF32:
        std::memcpy(out, src + first * 4, (size_t) count * 4);
        return GQ8_OK;
    case kF16:
        for (int64_t i = 0; i < count; ++i) {
            uint16_t h;
            std::memcpy(&h, src + (first + i) * 2, 2);
            out[i] = half_value(h);
        }
        return GQ8_OK;
    case kBF16:
        for (int64_t i = 0; i < count; ++i) {
            uint16_t h;
            std::memcpy(&h, src + (first + i) * 2, 2);
            const uint32_t bits = (uint32_t) h << 16;
            std::memcpy(&out[i], &bits, 4);
        }
        return GQ8_OK;
    case kF64:
        for (int64_t i = 0; i < count; ++i) {
            double d;
            std::memcpy(&d, src + (first + i) * 8, 8);
            out[i] = (float) d;
        }
        return GQ8_OK;
    default:
        return format_error("tensor '" + t.name + "' is " + dtype_name(t.dtype)
                            + ", not a floating-point tensor");
    }
}

// ---- config.json ------------------------------------------------------------
namespace {
int int_field(const Json &o, const char *key, int fallback, int *out)
{
    const Json *v = o.find(key);
    if (!v || v->kind == Json::Null) {
        *out = fallback;
        return GQ8_OK;
    }
    if (v->kind != Json::Number || !v->integral || v->integer < std::numeric_limits<int>::min()
        || v->integer > std::numeric_limits<int>::max())
        return format_error(std::string("config.json field '") + key + "' is not an int");
    *out = (int) v->integer;
    return GQ8_OK;
}

int double_field(const Json &o, const char *key, double fallback, double *out)
{
    const Json *v = o.find(key);
    if (!v || v->kind == Json::Null) {
        *out = fallback;
        return GQ8_OK;
    }
    if (v->kind != Json::Number)
        return format_error(std::string("config.json field '") + key + "' is not a number");
    *out = v->number;
    return GQ8_OK;
}

// A number, or a list whose first entry is taken (GemmaConfig.cpp:35-58).
int token_field(const Json &o, const char *key, int fallback, int *out)
{
    const Json *v = o.find(key);
    if (!v || v->kind == Json::Null) {
        *out = fallback;
        return GQ8_OK;
    }
    const Json *id = v;
    if (v->kind == Json::Array) {
        if (v->items.empty()) {
            *out = fallback;
            return GQ8_OK;
        }
        id = &v->items[0];
    }
    if (id->kind != Json::Number || !id->integral || id->integer < std::numeric_limits<int>::min()
        || id->integer > std::numeric_limits<int>::max())
        return format_error(std::string("config.json token id '") + key + "' is not an int");
    *out = (int) id->integer;
    return GQ8_OK;
}
} // namespace

int parse_gemma_config(const char *text, size_t length, GemmaConfigValues *out)
{
    Json root;
    JsonReader reader(text, length);
    if (!reader.read(root) || root.kind != Json::Object)
        return format_error("config.json is not a JSON object");
    if (const Json *t = root.find("model_type"); t && t->kind != Json::Null) {
        if (t->kind != Json::String)
            return format_error("config.json field 'model_type' is not a string");
        if (t->text != "gemma")
            return format_error("config.json describes a '" + t->text + "' model, not a gemma one");
    }
    GemmaConfigValues c;
    int s = GQ8_OK;
    if ((s = int_field(root, "vocab_size", c.vocab, &c.vocab))
        || (s = int_field(root, "hidden_size", c.width, &c.width))
        || (s = int_field(root, "intermediate_size", c.intermediate, &c.intermediate))
        || (s = int_field(root, "num_hidden_layers", c.layers, &c.layers))
        || (s = int_field(root, "num_attention_heads", c.heads, &c.heads))
        || (s = int_field(root, "num_key_value_heads", c.kv_heads, &c.kv_heads))
        || (s = int_field(root, "head_dim", c.head_dim, &c.head_dim))
        || (s = int_field(root, "max_position_embeddings", c.max_positions, &c.max_positions))
        || (s = double_field(root, "rms_norm_eps", c.rms_epsilon, &c.rms_epsilon))
        || (s = double_field(root, "rope_theta", c.rope_theta, &c.rope_theta))
        || (s = token_field(root, "bos_token_id", c.bos, &c.bos))
        || (s = token_field(root, "eos_token_id", c.eos, &c.eos))
        || (s = token_field(root, "pad_token_id", c.pad, &c.pad)))
        return s;
    if (const Json *t = root.find("tie_word_embeddings"); t && t->kind != Json::Null) {
        if (t->kind != Json::Bool)
            return format_error("config.json field 'tie_word_embeddings' is not a boolean");
        c.tied = t->boolean;
    }
    const std::pair<int, const char *> positive[] = {
        {c.vocab, "vocab_size"}, {c.width, "hidden_size"}, {c.intermediate, "intermediate_size"},
        {c.layers, "num_hidden_layers"}, {c.heads, "num_attention_heads"},
        {c.kv_heads, "num_key_value_heads"}, {c.head_dim, "head_dim"},
        {c.max_positions, "max_position_embeddings"}};
    for (const auto &p : positive)
        if (p.first <= 0)
            return format_error(std::string("config.json field '") + p.second + "' must be positive");
    if (!(c.rms_epsilon > 0.0))
        return format_error("config.json field 'rms_norm_eps' must be positive");
    if (!(c.rope_theta > 0.0))
        return format_error("config.json field 'rope_theta' must be positive");
    if (c.heads % c.kv_heads != 0)
        return format_error("config.json num_key_value_heads does not divide num_attention_heads");
    *out = c;
    return GQ8_OK;
}

} // namespace gq8

// ---- C ABI ------------------------------------------------------------------------

struct gq8_safetensors {
    std::unique_ptr<gq8::SafeTensorsFile> file;
};

const gq8::SafeTensorsFile *gq8::file_of(const gq8_safetensors *handle)
{
    return handle ? handle->file.get() : nullptr;
}

namespace {
int wrap(gq8::SafeTensorsFile *f, gq8_safetensors **out)
{
    *out = new gq8_safetensors{std::unique_ptr<gq8::SafeTensorsFile>(f)};
    return GQ8_OK;
}

const gq8::TensorInfo *tensor_at(const gq8_safetensors *f, int index)
{
    if (!f || index < 0 || index >= (int) f->file->tensors().size())
        return nullptr;
    return &f->file->tensors()[index];
}
} // namespace

extern "C" int gq8_safetensors_open(const char *path, gq8_safetensors **out)
{
    if (!path || !out)
        return gq8::report(GQ8_ERR_ARGUMENT, "safetensors_open: null argument");
    gq8::SafeTensorsFile *f = nullptr;
    if (int s = gq8::SafeTensorsFile::open(path, &f))
        return s;
    return wrap(f, out);
}

extern "C" int gq8_safetensors_from_bytes(const uint8_t *bytes, uint64_t size, gq8_safetensors **out)
{
    if ((!bytes && size) || !out)
        return gq8::report(GQ8_ERR_ARGUMENT, "safetensors_from_bytes: null argument");
    gq8::SafeTensorsFile *f = nullptr;
    if (int s = gq8::SafeTensorsFile::from_bytes(bytes, size, &f))
        return s;
    return wrap(f, out);
}

extern "C" void gq8_safetensors_close(gq8_safetensors *file)
{
    delete file;
}

extern "C" int gq8_safetensors_count(const gq8_safetensors *file)
{
    if (!file)
        return gq8::report(GQ8_ERR_ARGUMENT, "safetensors_count: null file");
    return (int) file->file->tensors().size();
}

extern "C" int gq8_safetensors_find(const gq8_safetensors *file, const char *name)
{
    if (!file || !name)
        return gq8::report(GQ8_ERR_ARGUMENT, "safetensors_find: null argument");
    const int i = file->file->find(name);
    return i >= 0 ? i : gq8::report(GQ8_ERR_FORMAT, std::string("no tensor named '") + name + "'");
}

extern "C" int gq8_safetensors_info(const gq8_safetensors *file, int index, const char **name,
                                    int *dtype, int *rank, int64_t *shape, int shape_capacity,
                                    uint64_t *byte_count)
{
    const gq8::TensorInfo *t = tensor_at(file, index);
    if (!t)
        return gq8::report(GQ8_ERR_ARGUMENT, "safetensors_info: no such tensor index");
    if (name)
        *name = t->name.c_str();
    if (dtype)
        *dtype = t->dtype;
    if (rank)
        *rank = (int) t->shape.size();
    if (shape)
        for (int i = 0; i < shape_capacity && i < (int) t->shape.size(); ++i)
            shape[i] = t->shape[i];
    if (byte_count)
        *byte_count = t->bytes;
    return GQ8_OK;
}

extern "C" int gq8_safetensors_read_floats(const gq8_safetensors *file, int index, int64_t first,
                                           int64_t count, float *out)
{
    const gq8::TensorInfo *t = tensor_at(file, index);
    if (!t || (!out && count > 0))
        return gq8::report(GQ8_ERR_ARGUMENT, "safetensors_read_floats: bad arguments");
    return file->file->read_floats(*t, first, count, out);
}

extern "C" const uint8_t *gq8_safetensors_raw(const gq8_safetensors *file, int index)
{
    const gq8::TensorInfo *t = tensor_at(file, index);
    return t ? file->file->blob_bytes(*t) : nullptr;
}

extern "C" int gq8_safetensors_metadata_count(const gq8_safetensors *file)
{
    if (!file)
        return gq8::report(GQ8_ERR_ARGUMENT, "safetensors_metadata_count: null file");
    return (int) file->file->metadata().size();
}

extern "C" int gq8_safetensors_metadata(const gq8_safetensors *file, int index, const char **key,
                                        const char **value)
{
    if (!file || index < 0 || index >= (int) file->file->metadata().size())
        return gq8::report(GQ8_ERR_ARGUMENT, "safetensors_metadata: no such entry");
    auto it = file->file->metadata().begin();
    std::advance(it, index);
    if (key)
        *key = it->first.c_str();
    if (value)
        *value = it->second.c_str();
    return GQ8_OK;
}

extern "C" int gq8_gemma_config_parse(const char *json_text, size_t length, int max_positions,
                                      int max_step_rows, gq8_shape *shape, gq8_token_ids *tokens)
{
    if (!json_text || !shape)
        return gq8::report(GQ8_ERR_ARGUMENT, "gemma_config_parse: null argument");
    gq8::GemmaConfigValues c;
    if (int s = gq8::parse_gemma_config(json_text, length, &c))
        return s;
    if (!c.tied)
        return gq8::report(GQ8_ERR_SHAPE, "this decoder ties the output projection to the embedding");
    gq8_shape out{};
    out.width = c.width;
    out.heads = c.heads;
    out.kv_heads = c.kv_heads;
    out.head_dim = c.head_dim;
    out.layers = c.layers;
    out.intermediate = c.intermediate;
    out.vocab = c.vocab;
    out.max_positions = max_positions > 0 ? std::min(max_positions, c.max_positions) : c.max_positions;
    out.max_step_rows = max_step_rows;
    out.rms_epsilon = (float) c.rms_epsilon;
    out.rope_theta = c.rope_theta;
    out.embedding_scale = std::sqrt((float) c.width); // GemmaConfig::embeddingScale
    *shape = out;
    if (tokens) {
        tokens->bos = c.bos;
        tokens->eos = c.eos;
        tokens->pad = c.pad;
    }
    return GQ8_OK;
}
