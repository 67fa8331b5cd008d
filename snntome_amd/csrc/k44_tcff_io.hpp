// k44_tcff_io.hpp — TCFF v1.0 plan file writer / reader (namespace k44_host).
//
// Byte format identical to the reference's wavec/k44_tcff_io.hpp:100-300 (writer) and accepted
// input identical to :319-428 (reader):
//   header (256-byte block): "II", u16 42, u32 first-IFD offset, "TCFFv1.0", u32 alignment (256),
//     u32 num_waves, u32 canvas_bytes (low 32 bits), u32 flags (bit0 trailing IFD hash,
//     bit2 canvas present), u64 FNV-1a-64 of header bytes [8, 32) at offset 32.
//   per K44_WAVE command: weight block (RDNA4 WMMA order), index block (u32), bias block (fp16),
//     each padded to 256; FNV-1a-64 over the three blocks; then a TIFF IFD with 21 tags
//     (+ 0x8444 geometry) and its out-of-line values; padded to 256.
// Build extension: tag 0x8445 (TCFF_WAVE_EXT, LONG x 12) is appended to a wave's IFD only when
// that wave needs it (row-index mode, or a canvas offset >= 2^32):
//   [idx_mode, idx_stride lo, idx_stride hi, x_base_off lo, hi, src_off lo, hi, y_off lo, hi,
//    res_off lo, hi, seg_len].
// The reference reader looks up tags 0x8440/0x8442/0x8443 only, so it ignores 0x8445.
// The reader here bounds-checks every offset it follows and returns false on any violation.
#pragma once
#include "k44_plan_types.hpp"

namespace k44_host {

static inline uint64_t fnv1a_hash64(const uint8_t *data, size_t len) {
    uint64_t h = 0xcbf29ce484222325ULL;
    for (const uint8_t *p = data, *e = data + len; p != e; ++p) h = (h ^ *p) * 0x100000001b3ULL;
    return h;
}

static inline uint32_t align_up_u32(uint32_t off, uint32_t align) {
    return (off + align - 1u) / align * align;
}

static constexpr uint16_t TIFF_BYTE = 1;
static constexpr uint16_t TIFF_ASCII = 2;
static constexpr uint16_t TIFF_SHORT = 3;
static constexpr uint16_t TIFF_LONG = 4;
static constexpr uint16_t TIFF_RATIONAL = 5;
static constexpr uint16_t TAG_TCFF_IMAGE_DEPTH = 0x80E5;
static constexpr uint16_t TAG_TCFF_WAVE_MAGIC = 0x8440;
static constexpr uint16_t TAG_TCFF_WAVE_PARAMS = 0x8441;
static constexpr uint16_t TAG_TCFF_AUX_OFFSETS = 0x8442;
static constexpr uint16_t TAG_TCFF_DATA_HASH64 = 0x8443;
static constexpr uint16_t TAG_TCFF_WAVE_GEOMETRY = 0x8444;
static constexpr uint16_t TAG_TCFF_WAVE_EXT = 0x8445;  // build extension
static constexpr uint32_t TCFF_MAGIC_WAVE = 0x45564157u;  // "WAVE"
static constexpr uint32_t TCFF_MAGIC_CANV = 0x564E4143u;  // "CANV"
static constexpr uint32_t TCFF_FLAG_TRAILING_IFD_HASH = 0x00000001u;
static constexpr uint32_t TCFF_FLAG_HAS_CANVAS = 0x00000004u;

struct TiffIFDEntry {
    uint16_t tag;
    uint16_t typ;
    uint32_t count;
    uint32_t val_or_off;
};

// Little-endian byte sink.
class TcffSink {
  public:
    std::vector<uint8_t> bytes;
    uint32_t size() const { return (uint32_t)bytes.size(); }
    void put(uint64_t v, int n) {
        for (int i = 0; i < n; ++i) bytes.push_back((uint8_t)(v >> (8 * i)));
    }
    void put_raw(const void *p, size_t n) {
        const uint8_t *b = (const uint8_t *)p;
        bytes.insert(bytes.end(), b, b + n);
    }
    void set_u32(uint32_t at, uint32_t v) {
        for (int i = 0; i < 4; ++i) bytes[at + i] = (uint8_t)(v >> (8 * i));
    }
    uint32_t align(uint32_t a) {
        bytes.resize(align_up_u32(size(), a), 0u);
        return size();
    }
};

static inline bool tcff_wave_needs_ext(const K44ExecCmd &c) {
    const uint64_t big = 1ULL << 32;
    return c.idx_mode != 0u || c.x_base_off >= big || c.src_off >= big || c.y_off >= big ||
           c.res_off >= big;
}

inline bool save_plan_to_tcff(const K44WavePlan &plan, const char *tcff_path,
                              const char *model_prefix = "K44Model", bool include_canvas = true,
                              bool include_geometry = true,
                              const uint16_t *live_canvas_f16 = nullptr) {
    (void)live_canvas_f16;
    std::vector<const K44ExecCmd *> waves;
    for (const auto &c : plan.cmds)
        if (c.type == K44CmdType::K44_WAVE) waves.push_back(&c);
    const uint32_t A = 256u;
    const uint32_t n_waves = (uint32_t)waves.size();
    const uint32_t canvas_bytes = (uint32_t)(plan.canvas_elems * 2u);
    const uint32_t pages = n_waves + (include_canvas ? 1u : 0u);
    const char *pfx = (model_prefix && model_prefix[0]) ? model_prefix : "K44Model";

    TcffSink out;
    out.bytes.reserve(plan.total_w_bytes + plan.total_idx_bytes + 65536u);
    out.put('I', 1);
    out.put('I', 1);
    out.put(42u, 2);
    out.put(0u, 4);
    out.put_raw("TCFFv1.0", 8);
    out.put(A, 4);
    out.put(n_waves, 4);
    out.put(canvas_bytes, 4);
    out.put(TCFF_FLAG_TRAILING_IFD_HASH | (include_canvas ? TCFF_FLAG_HAS_CANVAS : 0u), 4);
    out.put(fnv1a_hash64(out.bytes.data() + 8, 24), 8);
    out.align(A);

    uint32_t link_at = 4u;  // where the next IFD offset is patched in
    for (uint32_t wi = 0; wi < n_waves; ++wi) {
        const K44ExecCmd &c = *waves[wi];
        const uint32_t data_begin = out.size();
        const uint32_t w_off = out.size(), w_bytes = (uint32_t)(c.h_w_wmma.size() * 16u);
        out.put_raw(c.h_w_wmma.data(), w_bytes);
        out.align(A);
        const uint32_t i_off = out.size(), i_bytes = (uint32_t)(c.h_idx.size() * 4u);
        out.put_raw(c.h_idx.data(), i_bytes);
        out.align(A);
        const uint32_t b_off = out.size(), b_bytes = (uint32_t)(c.h_bias.size() * 2u);
        out.put_raw(c.h_bias.data(), b_bytes);
        out.align(A);
        const uint32_t data_end = out.size();
        const uint64_t h64 = fnv1a_hash64(out.bytes.data() + data_begin, data_end - data_begin);

        const uint32_t ifd_at = out.size();
        out.set_u32(link_at, ifd_at);
        const bool ext = tcff_wave_needs_ext(c);
        const uint16_t n_tags = (uint16_t)(21u + (include_geometry ? 1u : 0u) + (ext ? 1u : 0u));
        const uint32_t ext_base = ifd_at + 2u + 12u * n_tags + 4u;

        // Out-of-line values, each starting on an even offset.
        TcffSink tail;
        auto stash = [&](const void *p, size_t n) -> uint32_t {
            if (tail.size() & 1u) tail.put(0u, 1);
            const uint32_t at = ext_base + tail.size();
            tail.put_raw(p, n);
            return at;
        };
        auto stash_u32 = [&](std::initializer_list<uint32_t> v) -> uint32_t {
            std::vector<uint32_t> tmp(v);
            return stash(tmp.data(), tmp.size() * 4u);
        };
        auto lo = [](uint64_t v) { return (uint32_t)(v & 0xffffffffULL); };
        auto hi = [](uint64_t v) { return (uint32_t)(v >> 32); };

        char page[128], desc[320];
        std::snprintf(page, sizeof(page), "%s_Wave_%03u_%ux%u_S%u", pfx, wi, c.B, c.Cout,
                      c.cluster_size);
        std::snprintf(desc, sizeof(desc),
                      "TCFF %s Wave %u/%u | Cin=%u Cout=%u(log=%u) B=%u S=%u Act=%s Res=%d | "
                      "W=0x%x Idx=0x%x Bias=0x%x | FNV1a64=0x%016llx",
                      pfx, wi, n_waves, c.Cin, c.Cout, c.logical_Cout, c.B, c.cluster_size,
                      act_str(c.act), (int)c.has_residual, w_off, i_off, b_off,
                      (unsigned long long)h64);
        const uint32_t desc_len = (uint32_t)std::strlen(desc) + 1u;
        const uint32_t page_len = (uint32_t)std::strlen(page) + 1u;
        const uint32_t desc_at = stash(desc, desc_len);
        const uint32_t page_at = stash(page, page_len);
        const uint32_t rat_at = stash_u32({1u, 1u});
        const uint32_t par_at =
            stash_u32({c.Cin, c.Cout, c.B, c.cluster_size, c.weight_bits, 3u, (uint32_t)c.act,
                       (uint32_t)c.has_residual, c.h_out, c.w_out});
        const uint32_t aux_at = stash_u32({w_off, w_bytes, i_off, i_bytes, b_off, b_bytes,
                                           lo(c.src_off), lo(c.y_off), data_begin, data_end,
                                           lo(c.res_off)});
        const uint32_t hash_at = stash_u32({lo(h64), hi(h64)});
        uint32_t geo_at = 0u;
        if (include_geometry) {
            uint32_t g[10] = {3u, 1u, c.logical_Cout, c.h_out, c.w_out, c.Cout, 1u, 1u, 1u, 0u};
            auto it = plan.res_map.find(c.res_key_out);
            if (it != plan.res_map.end()) {
                const K44ResDesc &L = it->second;
                if (L.is_1d_tokens) {
                    const uint32_t toks = std::max(1u, c.w_out);
                    const uint32_t v[10] = {toks > 1u ? 2u : 1u, toks, c.logical_Cout, 1u, 1u, 1u,
                                            L.channel_stride, 1u, 1u, 0u};
                    std::memcpy(g, v, sizeof(g));
                } else {
                    const uint32_t v[10] = {3u, 1u, c.logical_Cout, c.h_out, c.w_out,
                                            c.Cout * L.channel_stride, L.channel_stride, L.W_pad,
                                            1u, L.W_pad + 4u};
                    std::memcpy(g, v, sizeof(g));
                }
            }
            geo_at = stash(g, sizeof(g));
        }
        uint32_t ext_at = 0u;
        if (ext)
            ext_at = stash_u32({c.idx_mode, lo(c.idx_stride), hi(c.idx_stride), lo(c.x_base_off),
                                hi(c.x_base_off), lo(c.src_off), hi(c.src_off), lo(c.y_off),
                                hi(c.y_off), lo(c.res_off), hi(c.res_off), c.seg_len});

        std::vector<TiffIFDEntry> tags = {{254, TIFF_LONG, 1, 2u},
                                          {256, TIFF_LONG, 1, c.B},
                                          {257, TIFF_LONG, 1, c.Cout},
                                          {258, TIFF_SHORT, 1, c.weight_bits},
                                          {259, TIFF_SHORT, 1, 1u},
                                          {262, TIFF_SHORT, 1, 1u},
                                          {266, TIFF_SHORT, 1, 1u},
                                          {270, TIFF_ASCII, desc_len, desc_at},
                                          {273, TIFF_LONG, 1, w_off},
                                          {277, TIFF_SHORT, 1, 1u},
                                          {278, TIFF_LONG, 1, c.Cout},
                                          {279, TIFF_LONG, 1, w_bytes},
                                          {282, TIFF_RATIONAL, 1, rat_at},
                                          {283, TIFF_RATIONAL, 1, rat_at},
                                          {285, TIFF_ASCII, page_len, page_at},
                                          {297, TIFF_SHORT, 2, wi | (pages << 16)},
                                          {339, TIFF_SHORT, 1, 3u},
                                          {TAG_TCFF_WAVE_MAGIC, TIFF_LONG, 1, TCFF_MAGIC_WAVE},
                                          {TAG_TCFF_WAVE_PARAMS, TIFF_LONG, 10, par_at},
                                          {TAG_TCFF_AUX_OFFSETS, TIFF_LONG, 11, aux_at},
                                          {TAG_TCFF_DATA_HASH64, TIFF_LONG, 2, hash_at}};
        if (include_geometry) tags.push_back({TAG_TCFF_WAVE_GEOMETRY, TIFF_LONG, 10, geo_at});
        if (ext) tags.push_back({TAG_TCFF_WAVE_EXT, TIFF_LONG, 12, ext_at});
        out.put(tags.size(), 2);
        for (const auto &t : tags) {
            out.put(t.tag, 2);
            out.put(t.typ, 2);
            out.put(t.count, 4);
            out.put(t.val_or_off, 4);
        }
        link_at = out.size();
        out.put(0u, 4);
        out.put_raw(tail.bytes.data(), tail.bytes.size());
        out.align(A);
    }

    FILE *fp = std::fopen(tcff_path, "wb");
    if (!fp) return false;
    const size_t n = std::fwrite(out.bytes.data(), 1, out.bytes.size(), fp);
    std::fclose(fp);
    return n == out.bytes.size();
}

static inline uint16_t read_u16_le(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t read_u32_le(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
           ((uint32_t)p[3] << 24);
}
static inline uint64_t read_u64_le(const uint8_t *p) {
    return (uint64_t)read_u32_le(p) | ((uint64_t)read_u32_le(p + 4) << 32);
}

// Loads weights, biases and (when the plan is single-frame and the canvas size matches the
// header) gather indices of every K44_WAVE command from a TCFF file into an already compiled
// plan, after verifying the header hash and every per-wave hash.
inline bool load_weights_from_tcff(K44WavePlan &plan, const char *tcff_path) {
    FILE *fp = std::fopen(tcff_path, "rb");
    if (!fp) {
        std::fprintf(stderr, "Failed to open TCFF file: %s\n", tcff_path);
        return false;
    }
    std::fseek(fp, 0, SEEK_END);
    const long fsz = std::ftell(fp);
    std::fseek(fp, 0, SEEK_SET);
    if (fsz < 256) {
        std::fclose(fp);
        return false;
    }
    std::vector<uint8_t> buf((size_t)fsz);
    const bool ok_read = std::fread(buf.data(), 1, buf.size(), fp) == buf.size();
    std::fclose(fp);
    if (!ok_read) return false;
    const uint8_t *B = buf.data();
    const uint64_t N = buf.size();
    auto in_file = [&](uint64_t off, uint64_t len) { return off <= N && len <= N - off; };

    if (B[0] != 'I' || B[1] != 'I' || read_u16_le(B + 2) != 42u) {
        std::fprintf(stderr, "Invalid TIFF header in TCFF file: %s\n", tcff_path);
        return false;
    }
    if (std::memcmp(B + 8, "TCFFv1.0", 8) != 0) {
        std::fprintf(stderr, "Invalid TCFFv1.0 magic in: %s\n", tcff_path);
        return false;
    }
    if (read_u64_le(B + 32) != fnv1a_hash64(B + 8, 24)) {
        std::fprintf(stderr, "Master header FNV-1a hash mismatch in: %s\n", tcff_path);
        return false;
    }
    const uint32_t file_canvas_bytes = read_u32_le(B + 24);
    const bool take_idx = plan.batch_size == 1u &&
                          (uint64_t)plan.canvas_elems * 2u == (uint64_t)file_canvas_bytes;
    std::vector<K44ExecCmd *> waves;
    for (auto &c : plan.cmds)
        if (c.type == K44CmdType::K44_WAVE) waves.push_back(&c);

    uint32_t ifd = read_u32_le(B + 4);
    size_t wi = 0;
    while (ifd != 0u && wi < waves.size()) {
        if (!in_file(ifd, 2)) return false;
        const uint16_t n_tags = read_u16_le(B + ifd);
        if (!in_file((uint64_t)ifd + 2u, 12ull * n_tags + 4u)) return false;
        uint32_t magic = 0u, aux_at = 0u, aux_n = 0u, hash_at = 0u;
        for (uint16_t t = 0; t < n_tags; ++t) {
            const uint8_t *e = B + ifd + 2u + 12u * t;
            const uint16_t tag = read_u16_le(e);
            if (tag == TAG_TCFF_WAVE_MAGIC) {
                magic = read_u32_le(e + 8);
            } else if (tag == TAG_TCFF_AUX_OFFSETS) {
                aux_n = read_u32_le(e + 4);
                aux_at = read_u32_le(e + 8);
            } else if (tag == TAG_TCFF_DATA_HASH64) {
                hash_at = read_u32_le(e + 8);
            }
        }
        const uint32_t next = read_u32_le(B + ifd + 2u + 12u * n_tags);
        if (magic == TCFF_MAGIC_CANV) {
            ifd = next;
            continue;
        }
        if (aux_at == 0u || aux_n < 10u || hash_at == 0u) return false;
        if (!in_file(aux_at, 40) || !in_file(hash_at, 8)) return false;
        const uint8_t *aux = B + aux_at;
        const uint32_t w_off = read_u32_le(aux + 0), w_bytes = read_u32_le(aux + 4);
        const uint32_t i_off = read_u32_le(aux + 8), i_bytes = read_u32_le(aux + 12);
        const uint32_t b_off = read_u32_le(aux + 16), b_bytes = read_u32_le(aux + 20);
        const uint32_t d0 = read_u32_le(aux + 32), d1 = read_u32_le(aux + 36);
        if (d1 < d0 || !in_file(d0, d1 - d0) || !in_file(w_off, w_bytes) ||
            !in_file(i_off, i_bytes) || !in_file(b_off, b_bytes))
            return false;
        if (read_u64_le(B + hash_at) != fnv1a_hash64(B + d0, d1 - d0)) {
            std::fprintf(stderr, "Wave %zu FNV-1a hash mismatch in: %s\n", wi, tcff_path);
            return false;
        }
        K44ExecCmd &c = *waves[wi];
        const size_t want_w = (size_t)c.Cout * c.B * 2u;
        c.h_w_wmma.assign(std::max(want_w, (size_t)w_bytes) / 16u, uint4_host{0u, 0u, 0u, 0u});
        std::memcpy(c.h_w_wmma.data(), B + w_off, std::min(want_w, (size_t)w_bytes));
        if (take_idx && i_bytes == c.h_idx.size() * 4u)
            std::memcpy(c.h_idx.data(), B + i_off, i_bytes);
        c.h_bias.assign(std::max<size_t>(c.Cout, b_bytes / 2u), 0u);
        std::memcpy(c.h_bias.data(), B + b_off, std::min((size_t)c.Cout * 2u, (size_t)b_bytes));
        ifd = next;
        ++wi;
    }
    return wi == waves.size();
}

}  // namespace k44_host
