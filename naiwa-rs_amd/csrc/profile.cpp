// The expert-cache profile reader (include/naiwa_policy.h): a ranked list of
// (layer, expert) pairs, best first, split per layer in rank order -- the
// reference's Profile::read (src/moe/profile.rs:50-97).  File layout (all
// little-endian): "STRP", five u32 (version 1, layers, experts, slots, n), then
// n pairs of u16 (layer, expert); a trailing rank table follows and is not read.
#include <cstdio>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/naiwa_moe.h"
#include "../../include/naiwa_policy.h"

struct naiwa_profile {
    std::vector<std::vector<uint32_t>> per_layer;
    uint32_t file_layers = 0, file_experts = 0, file_pairs = 0;
    int pairs = 0;
};

namespace {

uint32_t le32(const unsigned char* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
uint16_t le16(const unsigned char* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

} // namespace

extern "C" {

int naiwa_profile_read(const char* path, int num_layers, int num_experts, naiwa_profile** out) {
    if (!path || !out || num_layers <= 0 || num_experts <= 0) return NAIWA_E_INVALID;
    *out = nullptr;
    FILE* f = std::fopen(path, "rb");
    if (!f) return NAIWA_E_IO;
    unsigned char head[24];
    const size_t got = std::fread(head, 1, sizeof head, f);
    if (got < sizeof head || std::memcmp(head, "STRP", 4) != 0) {
        std::fclose(f);
        return NAIWA_E_FORMAT; // ProfileError::Magic
    }
    const uint32_t version = le32(head + 4), n = le32(head + 20);
    if (version != 1) {
        std::fclose(f);
        return NAIWA_E_UNSUPPORTED; // ProfileError::Version
    }
    std::vector<unsigned char> pairs;
    try {
        pairs.resize((size_t)n * 4);
    } catch (...) {
        std::fclose(f);
        return NAIWA_E_FORMAT; // cannot be a real file: treated as truncated
    }
    const size_t have = pairs.empty() ? 0 : std::fread(pairs.data(), 1, pairs.size(), f);
    std::fclose(f);
    if (have < pairs.size()) return NAIWA_E_FORMAT; // ProfileError::Truncated
    naiwa_profile* p = new (std::nothrow) naiwa_profile;
    if (!p) return NAIWA_E_NOMEM;
    try {
        p->per_layer.assign((size_t)num_layers, {});
        std::vector<char> seen((size_t)num_layers * num_experts, 0);
        for (uint32_t i = 0; i < n; ++i) {
            const int layer = le16(&pairs[4 * (size_t)i]), expert = le16(&pairs[4 * (size_t)i + 2]);
            if (layer >= num_layers || expert >= num_experts) continue;
            char& s = seen[(size_t)layer * num_experts + expert];
            if (s) continue;
            s = 1;
            p->per_layer[(size_t)layer].push_back((uint32_t)expert);
            ++p->pairs;
        }
    } catch (...) {
        delete p;
        return NAIWA_E_NOMEM;
    }
    p->file_layers = le32(head + 8);
    p->file_experts = le32(head + 12);
    p->file_pairs = n;
    *out = p;
    return NAIWA_OK;
}

int naiwa_profile_destroy(naiwa_profile* p) {
    delete p;
    return NAIWA_OK;
}

int naiwa_profile_layer(const naiwa_profile* p, int layer, uint32_t* experts, int capacity, int* n_out) {
    if (!p || !n_out || (capacity > 0 && !experts) || capacity < 0) return NAIWA_E_INVALID;
    *n_out = 0;
    if (layer < 0 || layer >= (int)p->per_layer.size()) return NAIWA_OK; // a layer the model lacks: empty
    const auto& v = p->per_layer[(size_t)layer];
    if ((int)v.size() > capacity) return NAIWA_E_INVALID;
    for (size_t i = 0; i < v.size(); ++i) experts[i] = v[i];
    *n_out = (int)v.size();
    return NAIWA_OK;
}

int naiwa_profile_info(const naiwa_profile* p, int* pairs, uint32_t* file_layers, uint32_t* file_experts,
                       uint32_t* file_pairs) {
    if (!p) return NAIWA_E_INVALID;
    if (pairs) *pairs = p->pairs;
    if (file_layers) *file_layers = p->file_layers;
    if (file_experts) *file_experts = p->file_experts;
    if (file_pairs) *file_pairs = p->file_pairs;
    return NAIWA_OK;
}

} // extern "C"
