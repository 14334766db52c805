// The packed model's metadata (manifest.json written by tools/repack.py:314-340), under
// the names and fields of the reference's src/model_info.h:38-204 (TensorInfo,
// ExpertPiece, ModelConfig, ModelInfo::load, getTensor, layer_file), read with this
// repository's own JSON reader; plus the per-layer file entries (file, size, stride,
// expert SHA-256s) and helpers that stream core.bin and layer_NN.bin into HipBackend
// buffers.
#pragma once
#include <cstdint>
#include <cstdio>
#include <fstream>
#include <map>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "json_reader.h"

namespace apex {

// One tensor inside core.bin (src/model_info.h:38-44).
struct TensorInfo {
    std::string dtype;
    std::vector<std::int64_t> shape;
    std::uint64_t offset = 0;
    std::uint64_t nbytes = 0;
};

// One piece of an expert slot (src/model_info.h:47-53).
struct ExpertPiece {
    std::string name;
    std::string dtype;
    std::vector<std::int64_t> shape;
    std::uint64_t offset = 0;
    std::uint64_t nbytes = 0;
};

// text_config values (src/model_info.h:56-80).
struct ModelConfig {
    int hidden_size = 0;
    int intermediate_size = 0;
    int moe_intermediate_size = 0;
    int num_attention_heads = 0;
    int num_key_value_heads = 0;
    int head_dim = 0;
    int num_hidden_layers = 0;
    int num_experts = 0;
    int top_k_experts = 0;
    int vocab_size = 0;
    int sliding_window = 0;
    double rms_norm_eps = 0;
    double final_logit_softcapping = 0;
    std::vector<std::string> layer_types;
    int global_head_dim = 0;
    int num_global_key_value_heads = 0;
    bool attention_k_eq_v = false;
    double rope_theta_sliding = 0;
    double rope_theta_full = 0;
    double partial_rotary_factor_full = 0;
};

// One layer_NN.bin entry of the manifest (tools/repack.py:237-257).
struct LayerFile {
    int layer = 0;
    std::string file;
    std::uint64_t size = 0;
    int num_experts = 0;
    std::uint64_t stride = 0;
    std::vector<std::string> expert_sha256;
};

struct ModelInfo {
    std::string dir;
    ModelConfig config;
    int quant_group_size = 0;
    int quant_bits = 0;
    std::string quant_mode;
    std::uint64_t core_size = 0;
    std::map<std::string, TensorInfo> core;
    std::uint64_t expert_slot_size = 0;               // the slot stride
    std::map<std::string, ExpertPiece> expert_pieces; // layout inside a slot
    std::vector<LayerFile> layers;

    const TensorInfo &getTensor(const std::string &name) const {
        auto it = core.find(name);
        if (it == core.end())
            throw std::runtime_error("tensor not found: " + name);
        return it->second;
    }
    const ExpertPiece &piece(const std::string &name) const {
        auto it = expert_pieces.find(name);
        if (it == expert_pieces.end())
            throw std::runtime_error("expert piece not found: " + name);
        return it->second;
    }

    static ModelInfo load(const std::string &dir);

    std::string layer_file(int layer) const {
        char filename[32];
        std::snprintf(filename, sizeof filename, "/layer_%02d.bin", layer);
        return dir + filename;
    }
};

inline ModelInfo ModelInfo::load(const std::string &dir) {
    std::ifstream in(dir + "/manifest.json");
    if (!in)
        throw std::runtime_error("ModelInfo: cannot open " + dir + "/manifest.json");
    std::stringstream ss;
    ss << in.rdbuf();
    const json::Value j = json::parse(ss.str());

    ModelInfo m;
    m.dir = dir;
    const json::Value &tc = j.at("text_config");
    ModelConfig &c = m.config;
    auto i = [&](const char *k) { return (int)tc.at(k).integer(); };
    c.hidden_size = i("hidden_size");
    c.intermediate_size = i("intermediate_size");
    c.moe_intermediate_size = i("moe_intermediate_size");
    c.num_attention_heads = i("num_attention_heads");
    c.num_key_value_heads = i("num_key_value_heads");
    c.head_dim = i("head_dim");
    c.num_hidden_layers = i("num_hidden_layers");
    c.num_experts = i("num_experts");
    c.top_k_experts = i("top_k_experts");
    c.vocab_size = i("vocab_size");
    c.sliding_window = i("sliding_window");
    c.rms_norm_eps = tc.at("rms_norm_eps").number();
    c.final_logit_softcapping = tc.at("final_logit_softcapping").number();
    for (const json::Value &t : tc.at("layer_types").array())
        c.layer_types.push_back(t.string());
    c.global_head_dim = i("global_head_dim");
    c.num_global_key_value_heads = i("num_global_key_value_heads");
    c.attention_k_eq_v = tc.at("attention_k_eq_v").boolean();
    const json::Value &rp = tc.at("rope_parameters");
    c.rope_theta_sliding = rp.at("sliding_attention").at("rope_theta").number();
    c.rope_theta_full = rp.at("full_attention").at("rope_theta").number();
    c.partial_rotary_factor_full = rp.at("full_attention").at("partial_rotary_factor").number();

    const json::Value &q = j.at("quantization");
    m.quant_group_size = (int)q.at("group_size").integer();
    m.quant_bits = (int)q.at("bits").integer();
    m.quant_mode = q.at("mode").string();

    auto shape_of = [](const json::Value &v) {
        std::vector<std::int64_t> s;
        for (const json::Value &d : v.array())
            s.push_back(d.integer());
        return s;
    };
    const json::Value &core = j.at("core");
    m.core_size = (std::uint64_t)core.at("size").integer();
    for (const json::Value &t : core.at("tensors").array()) {
        TensorInfo info;
        info.dtype = t.at("dtype").string();
        info.shape = shape_of(t.at("shape"));
        info.offset = (std::uint64_t)t.at("offset").integer();
        info.nbytes = (std::uint64_t)t.at("nbytes").integer();
        m.core.emplace(t.at("name").string(), std::move(info));
    }

    const std::vector<json::Value> &layers = j.at("layers").array();
    if (layers.empty())
        throw std::runtime_error("ModelInfo: manifest has no expert layers");
    for (const json::Value &l : layers) {
        LayerFile f;
        f.layer = (int)l.at("layer").integer();
        f.file = l.at("file").string();
        f.size = (std::uint64_t)l.at("size").integer();
        f.num_experts = (int)l.at("num_experts").integer();
        f.stride = (std::uint64_t)l.at("stride").integer();
        for (const json::Value &h : l.at("expert_sha256").array())
            f.expert_sha256.push_back(h.string());
        m.layers.push_back(std::move(f));
    }
    // all expert layers share one slot layout; read it from layer 0
    // (src/model_info.h:189-204)
    const json::Value &l0 = layers[0];
    m.expert_slot_size = (std::uint64_t)l0.at("stride").integer();
    for (const json::Value &p : l0.at("pieces").array()) {
        ExpertPiece piece;
        piece.name = p.at("name").string();
        piece.dtype = p.at("dtype").string();
        piece.shape = shape_of(p.at("shape"));
        piece.offset = (std::uint64_t)p.at("offset").integer();
        piece.nbytes = (std::uint64_t)p.at("nbytes").integer();
        const std::string name = piece.name;
        m.expert_pieces.emplace(name, std::move(piece));
    }
    return m;
}

} // namespace apex
