// gq8_gemma.cpp -- the model-directory runtime above the decoder: HF::Gemma's
// load / prepare / generate surface (Generation/Gemma.h:65-251) on the host.
//
// A Hugging Face Gemma directory is located the way ModelFiles::fromDirectory
// locates it (Model/ModelFiles.cpp:77-99), its config.json is read with
// generation_config.json's token ids applied over it (GemmaConfig.cpp:204-223),
// the tokenizer is required and checked against the embedding's vocabulary
// (Gemma.cpp:120-139) and every shard is mapped.  prepare() creates the
// decoder from the config and uploads the weights by checkpoint name;
// generate() is the decoder's greedy or sampled loop with the config's EOS,
// the token limit and the onToken callback.
#include "gemma_q8.h"
#include "gq8_checkpoint.hpp"
#include "gq8_json.hpp"

#include <algorithm>
#include <cstdlib>
#include <filesystem>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

namespace {
namespace fs = std::filesystem;

constexpr int kFileKinds = GQ8_FILE_SHARD;
const char *const kFileNames[kFileKinds] = {
    "config.json", "generation_config.json", "model.safetensors.index.json", "tokenizer.json",
    "tokenizer.model", "gemma-2b.gguf"};
constexpr const char *kWeightsName = "model.safetensors";
constexpr const char *kIndexName = "model.safetensors.index.json";

bool is_file(const fs::path &path)
{
    std::error_code error;
    return fs::is_regular_file(path, error);
}

int format(const std::string &message)
{
    return gq8::report(GQ8_ERR_FORMAT, message);
}

int read_text(const std::string &path, std::string *out)
{
    std::ifstream in(path, std::ios::binary);
    if (!in)
        return format("cannot read '" + path + "'");
    out->assign(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>());
    if (in.bad())
        return format("cannot read '" + path + "'");
    return GQ8_OK;
}

void copy_text(const std::string &text, char *out, size_t capacity, size_t *length)
{
    *length = text.size();
    if (out && capacity)
        std::copy_n(text.data(), std::min(capacity, text.size()), out);
}

// ShardIndex::fromJson (ShardIndex.cpp:31-74): weight_map an object of plain
// file names; each shard once, in the order the map first names it.
int shards_from_index(const std::string &text, std::vector<std::string> *names)
{
    gq8::Json root;
    gq8::JsonReader reader(text.data(), text.size());
    if (!reader.read(root) || root.kind != gq8::Json::Object)
        return format(std::string(kIndexName) + " is not a JSON object");
    const gq8::Json *map = root.find("weight_map");
    if (!map)
        return format(std::string(kIndexName) + " has no weight_map");
    if (map->kind != gq8::Json::Object)
        return format(std::string(kIndexName) + " weight_map is not an object");
    names->clear();
    for (const auto &[tensor, shard] : map->members) {
        if (shard.kind != gq8::Json::String)
            return format(std::string(kIndexName) + " maps '" + tensor
                          + "' to something that is not a file name");
        const std::string &file = shard.text;
        const bool plain = !file.empty() && file.find('/') == std::string::npos
                           && file.find('\\') == std::string::npos && file != "." && file != "..";
        if (!plain)
            return format(std::string(kIndexName) + " maps '" + tensor + "' to '" + file
                          + "', which is not a plain file name");
        if (std::find(names->begin(), names->end(), file) == names->end())
            names->push_back(file);
    }
    if (names->empty())
        return format(std::string(kIndexName) + " names no shards");
    if (const gq8::Json *meta = root.find("metadata"); meta && meta->kind != gq8::Json::Object)
        return format(std::string(kIndexName) + " metadata is not an object");
    return GQ8_OK;
}

// GenerationConfig::fromJson (GemmaConfig.cpp:87-101): each token id a number
// or the first of a list; an absent or null one leaves config.json's.
int apply_generation_config(const std::string &text, gq8_token_ids *ids)
{
    gq8::Json root;
    gq8::JsonReader reader(text.data(), text.size());
    if (!reader.read(root) || root.kind != gq8::Json::Object)
        return format("generation_config.json is not a JSON object");
    const std::pair<const char *, int *> fields[] = {
        {"bos_token_id", &ids->bos}, {"eos_token_id", &ids->eos}, {"pad_token_id", &ids->pad}};
    for (const auto &[key, slot] : fields) {
        const gq8::Json *v = root.find(key);
        if (!v || v->kind == gq8::Json::Null)
            continue;
        const gq8::Json *id = v;
        if (v->kind == gq8::Json::Array) {
            if (v->items.empty())
                continue;
            id = &v->items[0];
        }
        if (id->kind != gq8::Json::Number || !id->integral || id->integer < INT32_MIN
            || id->integer > INT32_MAX)
            return format(std::string("generation_config.json token id '") + key
                          + "' is not an int");
        *slot = (int) id->integer;
    }
    return GQ8_OK;
}
} // namespace

struct gq8_gemma {
    // ModelFiles: every path names a file that exists, or is empty
    std::string directory;
    std::string files[kFileKinds];
    std::vector<std::string> shards;
    std::string configText;
    gq8_shape config{};
    gq8_token_ids ids{};
    gq8_tokenizer *tokenizer = nullptr;
    std::vector<gq8_safetensors *> mapped;
    gq8_decoder *decoder = nullptr;
    int maximumTokens = 0;
    int promptCapacity = 512; // Gemma::defaultPromptCapacity (Gemma.h:235-251)
    gq8_sampling sampling{0.f, 0, 1.f, 0};
    gq8_token_callback onToken = nullptr;
    void *user = nullptr;
    gq8_run_stats last{};

    ~gq8_gemma() { unload(); }
    void unload()
    {
        if (decoder)
            gq8_decoder_destroy(decoder);
        decoder = nullptr;
        for (gq8_safetensors *f : mapped)
            gq8_safetensors_close(f);
        mapped.clear();
        if (tokenizer)
            gq8_tokenizer_destroy(tokenizer);
        tokenizer = nullptr;
        directory.clear();
        for (auto &f : files)
            f.clear();
        shards.clear();
        configText.clear();
    }
    bool loaded() const { return tokenizer != nullptr; }
};

extern "C" int gq8_gemma_create(gq8_gemma **out)
{
    if (!out)
        return gq8::report(GQ8_ERR_ARGUMENT, "gemma_create: null argument");
    *out = new gq8_gemma();
    return GQ8_OK;
}

extern "C" void gq8_gemma_destroy(gq8_gemma *g)
{
    if (!g)
        return;
    g->unload();
    delete g;
}

extern "C" int gq8_gemma_load(gq8_gemma *g, const char *model_directory)
{
    if (!g || !model_directory)
        return gq8::report(GQ8_ERR_ARGUMENT, "gemma_load: null argument");
    g->unload();
    gq8_gemma next;
    const fs::path dir(model_directory);
    std::error_code error;
    if (!fs::is_directory(dir, error))
        return format("'" + dir.string() + "' is not a directory");
    next.directory = dir.string();
    for (int k = 0; k < kFileKinds; ++k)
        if (is_file(dir / kFileNames[k]))
            next.files[k] = (dir / kFileNames[k]).string();
    auto missing = [&](const std::string &name) {
        return format("the model directory '" + dir.string() + "' has no " + name);
    };
    if (next.files[GQ8_FILE_CONFIG].empty())
        return missing(kFileNames[GQ8_FILE_CONFIG]);
    if (!next.files[GQ8_FILE_SHARD_INDEX].empty()) {
        std::string text;
        std::vector<std::string> names;
        if (int s = read_text(next.files[GQ8_FILE_SHARD_INDEX], &text))
            return s;
        if (int s = shards_from_index(text, &names))
            return s;
        for (const std::string &name : names) {
            if (!is_file(dir / name))
                return missing(name);
            next.shards.push_back((dir / name).string());
        }
    } else {
        if (!is_file(dir / kWeightsName))
            return missing(kWeightsName);
        next.shards.push_back((dir / kWeightsName).string());
    }

    // GemmaConfig::fromModelFiles, then the tokenizer it vouches for
    if (int s = read_text(next.files[GQ8_FILE_CONFIG], &next.configText))
        return s;
    if (int s = gq8_gemma_config_parse(next.configText.data(), next.configText.size(), 0, 0,
                                       &next.config, &next.ids))
        return s;
    if (!next.files[GQ8_FILE_GENERATION_CONFIG].empty()) {
        std::string text;
        if (int s = read_text(next.files[GQ8_FILE_GENERATION_CONFIG], &text))
            return s;
        if (int s = apply_generation_config(text, &next.ids))
            return s;
    }
    if (next.files[GQ8_FILE_TOKENIZER_JSON].empty())
        return format("the model directory " + dir.string()
                      + " has no tokenizer.json, and a string in and a string out needs one");
    if (int s = gq8_tokenizer_open(next.files[GQ8_FILE_TOKENIZER_JSON].c_str(), &next.tokenizer))
        return s;
    const int pieces = gq8_tokenizer_vocabulary_size(next.tokenizer);
    if (pieces > next.config.vocab)
        return format("this tokenizer names " + std::to_string(pieces)
                      + " tokens and config.json's embedding holds "
                      + std::to_string(next.config.vocab));
    for (const std::string &shard : next.shards) {
        gq8_safetensors *f = nullptr;
        if (int s = gq8_safetensors_open(shard.c_str(), &f))
            return s;
        next.mapped.push_back(f);
    }

    // nothing failed: take the located files over
    g->directory = std::move(next.directory);
    for (int k = 0; k < kFileKinds; ++k)
        g->files[k] = std::move(next.files[k]);
    g->shards = std::move(next.shards);
    g->configText = std::move(next.configText);
    g->config = next.config;
    g->ids = next.ids;
    g->tokenizer = next.tokenizer;
    next.tokenizer = nullptr;
    g->mapped = std::move(next.mapped);
    next.mapped.clear();
    g->maximumTokens = 0;
    return GQ8_OK;
}

extern "C" int gq8_gemma_directory_from_environment(char *out, size_t capacity, size_t *length)
{
    if (!length)
        return gq8::report(GQ8_ERR_ARGUMENT, "gemma_directory_from_environment: null length");
    const char *value = std::getenv("GEMMA_MODEL_DIR");
    copy_text(value ? std::string(value) : std::string(), out, capacity, length);
    return GQ8_OK;
}

extern "C" int gq8_gemma_is_loaded(const gq8_gemma *g)
{
    return g && g->loaded() ? 1 : 0;
}

extern "C" int gq8_gemma_is_prepared(const gq8_gemma *g)
{
    return g && g->decoder ? 1 : 0;
}

extern "C" int gq8_gemma_file(const gq8_gemma *g, int which, int index, char *out,
                              size_t capacity, size_t *length)
{
    if (!g || !length || which < 0 || which > GQ8_FILE_SHARD)
        return gq8::report(GQ8_ERR_ARGUMENT, "gemma_file: bad arguments");
    if (which == GQ8_FILE_SHARD) {
        if (index < 0 || index >= (int) g->shards.size())
            return gq8::report(GQ8_ERR_ARGUMENT, "gemma_file: no such shard");
        copy_text(g->shards[index], out, capacity, length);
    } else {
        copy_text(g->files[which], out, capacity, length);
    }
    return GQ8_OK;
}

extern "C" int gq8_gemma_shard_count(const gq8_gemma *g)
{
    return g ? (int) g->shards.size() : gq8::report(GQ8_ERR_ARGUMENT, "null gemma");
}

extern "C" int gq8_gemma_config(const gq8_gemma *g, gq8_shape *shape, gq8_token_ids *tokens)
{
    if (!g)
        return gq8::report(GQ8_ERR_ARGUMENT, "gemma_config: null gemma");
    if (!g->loaded())
        return gq8::report(GQ8_ERR_NOT_PREPARED, "this Gemma has not loaded a model yet");
    if (shape)
        *shape = g->config;
    if (tokens)
        *tokens = g->ids;
    return GQ8_OK;
}

extern "C" int gq8_gemma_set_maximum_tokens(gq8_gemma *g, int count)
{
    if (!g)
        return gq8::report(GQ8_ERR_ARGUMENT, "null gemma");
    if (count < 0)
        return gq8::report(GQ8_ERR_ARGUMENT,
                           "a token limit is a count, or zero for the window's own bound, and "
                           "this one is " + std::to_string(count));
    g->maximumTokens = count;
    return GQ8_OK;
}

extern "C" int gq8_gemma_maximum_tokens(const gq8_gemma *g)
{
    return g ? g->maximumTokens : gq8::report(GQ8_ERR_ARGUMENT, "null gemma");
}

extern "C" int gq8_gemma_set_prompt_capacity(gq8_gemma *g, int rows)
{
    if (!g)
        return gq8::report(GQ8_ERR_ARGUMENT, "null gemma");
    if (rows <= 0)
        return gq8::report(GQ8_ERR_ARGUMENT, "a prefill block has to carry at least one row");
    g->promptCapacity = rows;
    return GQ8_OK;
}

extern "C" int gq8_gemma_prompt_capacity(const gq8_gemma *g)
{
    return g ? g->promptCapacity : gq8::report(GQ8_ERR_ARGUMENT, "null gemma");
}

extern "C" int gq8_gemma_set_sampling(gq8_gemma *g, const gq8_sampling *options)
{
    if (!g || !options)
        return gq8::report(GQ8_ERR_ARGUMENT, "gemma_set_sampling: null argument");
    if (int s = gq8::check_sampling(*options))
        return s;
    g->sampling = *options;
    if (g->decoder)
        return gq8_decoder_set_sampling(g->decoder, &g->sampling);
    return GQ8_OK;
}

extern "C" int gq8_gemma_set_on_token(gq8_gemma *g, gq8_token_callback on_token, void *user)
{
    if (!g)
        return gq8::report(GQ8_ERR_ARGUMENT, "null gemma");
    g->onToken = on_token;
    g->user = user;
    return GQ8_OK;
}

extern "C" int gq8_gemma_prepare(gq8_gemma *g)
{
    if (!g)
        return gq8::report(GQ8_ERR_ARGUMENT, "null gemma");
    if (!g->loaded())
        return gq8::report(GQ8_ERR_NOT_PREPARED, "this Gemma has not loaded a model yet");
    if (g->decoder)
        gq8_decoder_destroy(g->decoder);
    g->decoder = nullptr;
    gq8_shape shape = g->config;
    shape.max_step_rows = std::min(g->promptCapacity, shape.max_positions);
    if (int s = gq8_shape_validate(&shape))
        return s;
    gq8_decoder *d = nullptr;
    if (int s = gq8_decoder_create(&shape, &d))
        return s;
    int s = gq8_decoder_load_safetensors(d, g->mapped.data(), (int) g->mapped.size());
    if (s == GQ8_OK)
        s = gq8_decoder_set_sampling(d, &g->sampling);
    if (s != GQ8_OK) {
        gq8_decoder_destroy(d);
        return s;
    }
    g->decoder = d;
    return GQ8_OK;
}

extern "C" gq8_decoder *gq8_gemma_decoder(gq8_gemma *g)
{
    return g ? g->decoder : nullptr;
}

extern "C" const gq8_tokenizer *gq8_gemma_tokenizer(const gq8_gemma *g)
{
    return g ? g->tokenizer : nullptr;
}

namespace {
// Gemma::generate (Gemma.cpp:402-457) into `ids`: the count or a status.
int run(gq8_gemma *g, const int32_t *prompt, int prompt_length, std::vector<int32_t> *ids)
{
    if (!g->decoder)
        return gq8::report(GQ8_ERR_NOT_PREPARED, "this Gemma has not been prepared on a device yet");
    if (!prompt && prompt_length > 0)
        return gq8::report(GQ8_ERR_ARGUMENT, "gemma_generate: null prompt");
    const int window = g->config.max_positions - std::max(prompt_length, 0);
    const int limit = g->maximumTokens > 0 ? std::min(g->maximumTokens, window) : window;
    ids->assign((size_t) std::max(limit, 1), 0);
    const int32_t none = 0;
    gq8_run_stats stats{};
    const int count = gq8_generate_streaming(g->decoder, prompt ? prompt : &none, prompt_length,
                                             g->maximumTokens, g->ids.eos, 1, ids->data(), &stats,
                                             g->onToken, g->user);
    if (count < 0)
        return count;
    g->last = stats;
    ids->resize((size_t) count);
    return count;
}

// Tokenizer::encodeWithBos of the text (Gemma.cpp:596-603)
int encode_with_bos(const gq8_gemma *g, const char *text, size_t length,
                    std::vector<int32_t> *prompt)
{
    const int n = gq8_tokenizer_encode(g->tokenizer, text, length, 1, nullptr, 0);
    if (n < 0)
        return n;
    prompt->assign((size_t) std::max(n, 1), 0);
    if (int s = gq8_tokenizer_encode(g->tokenizer, text, length, 1, prompt->data(), n); s < 0)
        return s;
    prompt->resize((size_t) n);
    return n;
}
} // namespace

extern "C" int gq8_gemma_generate(gq8_gemma *g, const int32_t *prompt, int prompt_length,
                                  int32_t *out, int capacity)
{
    if (!g || (!out && capacity > 0) || capacity < 0)
        return gq8::report(GQ8_ERR_ARGUMENT, "gemma_generate: bad arguments");
    std::vector<int32_t> ids;
    const int count = run(g, prompt, prompt_length, &ids);
    if (count > 0)
        std::copy_n(ids.begin(), std::min(count, capacity), out);
    return count;
}

extern "C" int gq8_gemma_generate_from_text(gq8_gemma *g, const char *text, size_t length,
                                            int32_t *out, int capacity)
{
    if (!g || (!text && length) || (!out && capacity > 0) || capacity < 0)
        return gq8::report(GQ8_ERR_ARGUMENT, "gemma_generate_from_text: bad arguments");
    if (!g->decoder)
        return gq8::report(GQ8_ERR_NOT_PREPARED, "this Gemma has not been prepared on a device yet");
    std::vector<int32_t> prompt, ids;
    if (int s = encode_with_bos(g, text, length, &prompt); s < 0)
        return s;
    const int count = run(g, prompt.data(), (int) prompt.size(), &ids);
    if (count > 0)
        std::copy_n(ids.begin(), std::min(count, capacity), out);
    return count;
}

extern "C" int gq8_gemma_generate_text(gq8_gemma *g, const char *text, size_t length, char *out,
                                       size_t capacity, size_t *out_length)
{
    if (!g || (!text && length) || !out_length)
        return gq8::report(GQ8_ERR_ARGUMENT, "gemma_generate_text: bad arguments");
    if (!g->decoder)
        return gq8::report(GQ8_ERR_NOT_PREPARED, "this Gemma has not been prepared on a device yet");
    std::vector<int32_t> prompt, ids;
    if (int s = encode_with_bos(g, text, length, &prompt); s < 0)
        return s;
    const int count = run(g, prompt.data(), (int) prompt.size(), &ids);
    if (count < 0)
        return count;
    return gq8_tokenizer_decode(g->tokenizer, ids.data(), count, 0, out, capacity, out_length);
}

extern "C" int gq8_gemma_text_for_tokens(const gq8_gemma *g, const int32_t *tokens, int count,
                                         char *out, size_t capacity, size_t *length)
{
    if (!g)
        return gq8::report(GQ8_ERR_ARGUMENT, "null gemma");
    if (!g->loaded())
        return gq8::report(GQ8_ERR_NOT_PREPARED, "this Gemma has not loaded a model yet");
    return gq8_tokenizer_decode(g->tokenizer, tokens, count, 0, out, capacity, length);
}

extern "C" int gq8_gemma_last_stats(const gq8_gemma *g, gq8_run_stats *stats)
{
    if (!g || !stats)
        return gq8::report(GQ8_ERR_ARGUMENT, "gemma_last_stats: null argument");
    *stats = g->last;
    return GQ8_OK;
}
