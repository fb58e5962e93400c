// packed_checkpoint.hpp -- the packed checkpoint on disk: the group-64 wire
// layout of packed.rs in per-layer files plus embedding, readout and norm
// files, described by a `packed-<format>.json` manifest.
//
//   written by  export_packed.rs:13-103 (export_webgpu_packed)
//   validated   prepare_hf_q4.py:65-114 (detect_format, validate_packed,
//               verify_files, checked_file), same checks and messages
//   read by     browser/pplx.rs:140-330 (manifest, embedding rows, readout)
//
// PackedCheckpoint::open validates the manifest against its own source
// tensor index and the expected model shape, then checks every listed file's
// size and SHA-256. Reads return the packed bytes of a tensor, of embedding
// rows (the EmbeddingCache source, browser/pplx.rs:76-137) or of the readout
// and norm files. Failures are INVALID_CHECKPOINT errors carrying the
// validator's message.
#pragma once

#include <sys/stat.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <map>
#include <regex>
#include <set>
#include <string>
#include <vector>

#include "inference.hpp"
#include "json.hpp"
#include "sha256.hpp"

namespace decisive {

struct PackedFormat {
    std::string name;    // "q4-e4" or "q8-e8"
    std::string scheme;  // prepare_hf_q4.py:15-20
    int bits;
    size_t group_bytes;
};

inline const std::vector<PackedFormat> &packed_formats() {
    static const std::vector<PackedFormat> f = {{"q4-e4", "q4-w4a8-e4-r4-g64", 4, 36},
                                                {"q8-e8", "q8-w8a8-e8-r8-g64", 8, 68}};
    return f;
}

struct PackedTensor {
    std::string name;
    std::vector<uint64_t> shape;
    uint64_t start = 0, end = 0;
};

struct PackedLayer {
    std::string file;
    uint64_t bytes = 0;
    std::vector<PackedTensor> tensors;
};

// The model a checkpoint must describe. Defaults are the pinned Pplx source
// (examples/pplx-flash/model.json revision; 32 decoder layers, hidden 2560,
// 255 readout codes, 2 source shards).
struct PackedModel {
    std::string revision = "6d771ad7b5ecff5e93b8fc7b90d4c5ccc341954d";
    size_t layers = 32;
    size_t hidden = 2560;
    size_t readout_rows = 255;
    size_t shards = 2;
};

class PackedCheckpoint {
public:
    // prepare_hf_q4.py:58-62 packed_size
    static Result<uint64_t> packed_size(const std::vector<uint64_t> &shape, size_t group_bytes) {
        uint64_t n = 1;
        for (uint64_t d : shape) n *= d;
        if (shape.size() == 2) {
            if (shape[1] % 64 != 0) return invalid("Matrix width is not a multiple of 64");
            return n / 64 * group_bytes;
        }
        return n * 2;
    }

    // prepare_hf_q4.py:38-42 checked_file: a plain name of a regular file in dir.
    static Result<std::string> checked_file(const std::string &dir, const std::string &name) {
        static const std::regex safe("[a-zA-Z0-9_.-]+");
        if (!std::regex_match(name, safe) || name == "." || name == "..") return invalid("Unsafe filename");
        std::string path = dir + "/" + name;
        struct stat st;
        if (lstat(path.c_str(), &st) != 0 || !S_ISREG(st.st_mode))
            return invalid("Missing file or symlink: " + name);
        return path;
    }

    // prepare_hf_q4.py:45-48 verify_files: size and SHA-256 of every file.
    static Status verify_files(const std::string &dir, const Json &files) {
        if (!files.is_object()) return invalid("Unexpected packed files");
        for (const auto &kv : files.as_object()) {
            auto path = checked_file(dir, kv.first);
            if (!path) return path.error();
            std::ifstream f(path.value(), std::ios::binary);
            Sha256 h;
            std::vector<char> buf(1 << 20);
            uint64_t bytes = 0;
            while (f) {
                f.read(buf.data(), (std::streamsize)buf.size());
                std::streamsize got = f.gcount();
                if (got <= 0) break;
                h.update(buf.data(), (size_t)got);
                bytes += (uint64_t)got;
            }
            const Json &want = kv.second;
            if (!want["bytes"].is_number() || (uint64_t)want["bytes"].as_number() != bytes ||
                !want["sha256"].is_string() || want["sha256"].as_string() != h.hex())
                return invalid("Checksum or size mismatch: " + kv.first);
        }
        return {};
    }

    // prepare_hf_q4.py:65-68 detect_format: exactly one packed manifest.
    static Result<PackedFormat> detect_format(const std::string &dir) {
        std::vector<PackedFormat> found;
        for (const PackedFormat &f : packed_formats()) {
            struct stat st;
            if (stat((dir + "/packed-" + f.name + ".json").c_str(), &st) == 0) found.push_back(f);
        }
        if (found.size() != 1) return invalid("Expected exactly one packed manifest");
        return found[0];
    }

    // prepare_hf_q4.py:71-114 validate_packed + verify_files. `verify_digests`
    // false skips the SHA-256 pass (sizes are still checked by the layout).
    static Result<PackedCheckpoint> open(const std::string &dir, const PackedModel &model = PackedModel{},
                                         bool verify_digests = true) {
        auto format = detect_format(dir);
        if (!format) return format.error();
        const PackedFormat &fmt = format.value();
        auto mpath = checked_file(dir, "packed-" + fmt.name + ".json");
        if (!mpath) return mpath.error();
        Json parsed;
        try {
            parsed = Json::parse(slurp(mpath.value()));
        } catch (const std::exception &e) {
            return invalid(std::string("Invalid packed manifest: ") + e.what());
        }
        const Json &m = parsed;
        PackedCheckpoint c;
        c.dir_ = dir;
        c.format_ = fmt;
        c.model_ = model;
        const size_t group = fmt.group_bytes;
        if (!(num(m["schema_version"]) == 1 && m["scheme"] == Json(fmt.scheme))) return invalid("Unsupported packed format");
        if (!(m["revision"] == Json(model.revision))) return invalid("Wrong source revision");
        if (!(num(m["group_size"]) == 64 && num(m["group_bytes"]) == (double)group &&
              num(m["embedding_row_bytes"]) == (double)(model.hidden / 64 * group)))
            return invalid("Wrong group layout");
        c.row_bytes_ = model.hidden / 64 * group;
        if (!(m["layers"].is_array() && m["layers"].size() == model.layers && m["headers"].is_array() &&
              m["headers"].size() == model.shards))
            return invalid("Incomplete checkpoint");
        // the source tensor index: every tensor BF16 and named once
        std::map<std::string, std::vector<uint64_t>> source;
        for (const Json &h : m["headers"].as_array()) {
            Json idx;
            try {
                idx = Json::parse(h.is_string() ? h.as_string() : std::string("null"));
            } catch (const std::exception &) {
                return invalid("Invalid source tensor index");
            }
            if (!idx.is_object()) return invalid("Invalid source tensor index");
            for (const auto &kv : idx.as_object()) {
                if (kv.first == "__metadata__") continue;
                auto shape = shape_of(kv.second["shape"]);
                if (source.count(kv.first) || !(kv.second["dtype"] == Json("BF16")) || !shape)
                    return invalid("Invalid source tensor index");
                source[kv.first] = shape.value();
            }
        }
        std::set<std::string> expected_files;
        uint64_t decoder = 0;
        const Json &files = m["files"];
        if (!files.is_object()) return invalid("Unexpected packed files");
        for (size_t index = 0; index < model.layers; index++) {
            const Json &layer = m["layers"][index];
            char want[64];
            snprintf(want, sizeof want, "%s-layer-%02zu.bin", fmt.name.c_str(), index);
            if (!(layer["file"] == Json(want))) return invalid("Wrong layer filename/order");
            expected_files.insert(want);
            const std::string prefix = "language_model.layers." + std::to_string(index) + ".";
            std::set<std::string> expected, seen;
            for (const auto &kv : source)
                if (kv.first.compare(0, prefix.size(), prefix) == 0) expected.insert(kv.first);
            PackedLayer pl;
            pl.file = want;
            uint64_t position = 0;
            if (!layer["tensors"].is_array()) return invalid("Missing layer tensors");
            for (const Json &t : layer["tensors"].as_array()) {
                const std::string key = t["name"].is_string() ? t["name"].as_string() : std::string();
                if (!expected.count(key) || seen.count(key)) return invalid("Unknown or repeated tensor");
                seen.insert(key);
                auto shape = shape_of(t["shape"]);
                if (!shape || shape.value() != source[key]) return invalid("Tensor shape mismatch");
                auto size = packed_size(shape.value(), group);
                if (!size) return size.error();
                if (!(num(t["start"]) == (double)position && num(t["end"]) - (double)position == (double)size.value()))
                    return invalid("Invalid tensor range");
                pl.tensors.push_back(PackedTensor{key, shape.value(), position, position + size.value()});
                position += size.value();
            }
            if (seen != expected || seen.empty()) return invalid("Missing layer tensors");
            if (!(num(layer["bytes"]) == (double)position && num(files[want]["bytes"]) == (double)position))
                return invalid("Layer size mismatch");
            pl.bytes = position;
            decoder += position;
            c.layers_.push_back(std::move(pl));
        }
        if (!(num(m["decoder_bytes"]) == (double)decoder)) return invalid("Decoder total mismatch");
        auto embed = source.find("language_model.embed_tokens.weight");
        if (embed == source.end() || embed->second.size() != 2 || embed->second[1] != model.hidden)
            return invalid("Invalid embedding payload");
        c.vocab_ = embed->second[0];
        auto embed_size = packed_size(embed->second, group);
        if (!embed_size) return embed_size.error();
        struct Aux {
            const char *key;
            uint64_t size;
            std::string *file;
        } aux[3] = {{"embedding", embed_size.value(), &c.embedding_},
                    {"readout", model.readout_rows * (model.hidden / 64) * group, &c.readout_},
                    {"norm", model.hidden * 2, &c.norm_}};
        for (Aux &a : aux) {
            const std::string want = fmt.name + "-" + a.key + ".bin";
            if (!(m[a.key] == Json(want)) || !(num(files[want]["bytes"]) == (double)a.size))
                return invalid(std::string("Invalid ") + a.key + " payload");
            *a.file = want;
            expected_files.insert(want);
        }
        std::set<std::string> listed;
        for (const auto &kv : files.as_object()) listed.insert(kv.first);
        if (listed != expected_files) return invalid("Unexpected packed files");
        if (verify_digests) {
            Status s = verify_files(dir, files);
            if (!s) return s.error();
        } else {
            for (const auto &kv : files.as_object()) {
                auto path = checked_file(dir, kv.first);
                if (!path) return path.error();
            }
        }
        c.manifest_ = m;
        return c;
    }

    const PackedFormat &format() const { return format_; }
    const PackedModel &model() const { return model_; }
    const std::vector<PackedLayer> &layers() const { return layers_; }
    const Json &manifest() const { return manifest_; }
    size_t row_bytes() const { return row_bytes_; }
    uint64_t vocab() const { return vocab_; }
    // dz_layout of the 2-D tensors, embedding rows and readout
    int32_t layout() const { return format_.bits == 4 ? 0 /* DZ_Q4_G64_F32 */ : 1 /* DZ_Q8_G64_F32 */; }

    // The packed bytes of one layer tensor (2-D: wire layout; else BF16).
    Result<std::vector<uint8_t>> tensor(size_t layer, const std::string &name) const {
        if (layer >= layers_.size()) return invalid("layer index out of range");
        for (const PackedTensor &t : layers_[layer].tensors)
            if (t.name == name) return read(layers_[layer].file, t.start, t.end - t.start);
        return invalid("missing tensor " + name);
    }

    // Packed embedding rows of `ids`, in order (browser/pplx.rs:76-137 reads
    // them from the embedding file at id * row_bytes).
    Result<std::vector<uint8_t>> embedding_rows(const std::vector<uint32_t> &ids) const {
        std::vector<uint8_t> out(ids.size() * row_bytes_);
        auto path = checked_file(dir_, embedding_);
        if (!path) return path.error();
        std::ifstream f(path.value(), std::ios::binary);
        for (size_t i = 0; i < ids.size(); i++) {
            if (ids[i] >= vocab_) return Error("INVALID_REQUEST", "token out of range");
            f.seekg((std::streamoff)((uint64_t)ids[i] * row_bytes_));
            f.read((char *)out.data() + i * row_bytes_, (std::streamsize)row_bytes_);
            if ((size_t)f.gcount() != row_bytes_) return invalid("Incomplete embedding row");
        }
        return out;
    }

    // The answer temperature of decision_config.json, when the checkpoint
    // directory holds it (prepare_hf_q4.py copies it there; input.rs:127-131
    // requires it finite and positive).
    Result<float> temperature() const {
        auto path = checked_file(dir_, "decision_config.json");
        if (!path) return path.error();
        Json d;
        try {
            d = Json::parse(slurp(path.value()));
        } catch (const std::exception &e) {
            return invalid(std::string("Invalid decision config: ") + e.what());
        }
        const Json &t = static_cast<const Json &>(d)["temperature"];
        const float v = t.is_number() ? (float)t.as_number() : NAN;
        if (!(std::isfinite(v) && v > 0.0f)) return Error::engine("invalid temperature");
        return v;
    }

    Result<std::vector<uint8_t>> readout_bytes() const {
        return read(readout_, 0, model_.readout_rows * row_bytes_);
    }

    // The final norm weights (BF16 on disk) as f32.
    Result<std::vector<float>> norm() const {
        auto raw = read(norm_, 0, model_.hidden * 2);
        if (!raw) return raw.error();
        std::vector<float> out(model_.hidden);
        for (size_t i = 0; i < out.size(); i++) {
            uint32_t bits = (uint32_t)(raw.value()[2 * i] | raw.value()[2 * i + 1] << 8) << 16;
            memcpy(&out[i], &bits, 4);
        }
        return out;
    }

private:
    static Error invalid(const std::string &message) { return Error("INVALID_CHECKPOINT", message); }
    static std::string slurp(const std::string &path) {
        std::ifstream f(path, std::ios::binary);
        return std::string((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    }
    static double num(const Json &v) { return v.is_number() ? v.as_number() : -1.0; }
    static Result<std::vector<uint64_t>> shape_of(const Json &v) {
        if (!v.is_array()) return invalid("Invalid source tensor index");
        std::vector<uint64_t> s;
        for (const Json &d : v.as_array()) {
            if (!d.is_number() || d.as_number() < 0 || d.as_number() != (double)(uint64_t)d.as_number())
                return invalid("Invalid source tensor index");
            s.push_back((uint64_t)d.as_number());
        }
        return s;
    }

    Result<std::vector<uint8_t>> read(const std::string &file, uint64_t start, uint64_t bytes) const {
        auto path = checked_file(dir_, file);
        if (!path) return path.error();
        std::ifstream f(path.value(), std::ios::binary);
        std::vector<uint8_t> out(bytes);
        f.seekg((std::streamoff)start);
        f.read((char *)out.data(), (std::streamsize)bytes);
        if ((uint64_t)f.gcount() != bytes) return invalid("Checksum or size mismatch: " + file);
        return out;
    }

    std::string dir_;
    PackedFormat format_;
    PackedModel model_;
    std::vector<PackedLayer> layers_;
    std::string embedding_, readout_, norm_;
    size_t row_bytes_ = 0;
    uint64_t vocab_ = 0;
    Json manifest_;
};

}  // namespace decisive
