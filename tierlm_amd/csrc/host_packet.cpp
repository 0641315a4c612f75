/* host_packet.cpp - reader of the reference's compiled model stores: the
 * manifest (<name>.tlmm) and the per-drive packet files (<dir>/<name>.tlmp),
 * src/lib/tlm_packet.h:8-151 and the format described at
 * src/lib/tlm_packet.c:8-34.  Read-only: the writer (the compiler) is not part
 * of this library.
 *
 * Every check of the reference's loader is made (src/lib/tlm_packet.c:673-751,
 * 211-275, 788-815, 877-917): one valid layout, header CRC32C, packet table
 * SHA-256, report CRC32C, record ranges, strict order, no overlapping
 * extents, packet header / length / payload CRC32C on every read, tensor
 * directory bounds.  CRC32C (Castagnoli, reflected polynomial 0x82F63B78) and
 * SHA-256 (FIPS 180-4) are written from their published definitions. */
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <memory>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/tlm_hip.h"

int tlmh_seterr(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

namespace {

constexpr uint32_t MANIFEST_MAGIC = 0x4D4D4C54u;   /* "TLMM" */
constexpr uint32_t PACKET_MAGIC = 0x504D4C54u;     /* "TLMP" */
constexpr uint32_t STORE_VERSION = 2u;
constexpr uint32_t FIXED = 512u, CRC_AT = 508u, DRIVE_BYTES = 256u, REC_BYTES = 48u, HDR_BYTES = 64u;
constexpr uint32_t MAX_DRIVES = 16u, MAX_PACKETS = 1u << 24;
constexpr uint64_t MAX_REPORT = 64ull << 20, MAX_PAYLOAD = 1ull << 40, ALIGN_IO = 4096u, ALIGN_DIR = 64u;
constexpr uint16_t KNOWN_FLAGS = 0x3u;

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
uint64_t rd64(const uint8_t *p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }
float rdf(const uint8_t *p) {
    uint32_t u = rd32(p);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ---- CRC32C, slicing by 8 ------------------------------------------------- */
struct Crc32c {
    uint32_t t[8][256];
    Crc32c() {
        for (uint32_t i = 0; i < 256; i++) {
            uint32_t c = i;
            for (int k = 0; k < 8; k++) c = (c >> 1) ^ (0x82F63B78u & (0u - (c & 1u)));
            t[0][i] = c;
        }
        for (uint32_t i = 0; i < 256; i++)
            for (int s = 1; s < 8; s++) t[s][i] = (t[s - 1][i] >> 8) ^ t[0][t[s - 1][i] & 0xFF];
    }
    uint32_t operator()(uint32_t crc, const uint8_t *p, size_t n) const {
        uint32_t c = ~crc;
        while (n >= 8) {
            const uint32_t lo = rd32(p) ^ c, hi = rd32(p + 4);
            c = t[7][lo & 0xFF] ^ t[6][(lo >> 8) & 0xFF] ^ t[5][(lo >> 16) & 0xFF] ^ t[4][lo >> 24] ^
                t[3][hi & 0xFF] ^ t[2][(hi >> 8) & 0xFF] ^ t[1][(hi >> 16) & 0xFF] ^ t[0][hi >> 24];
            p += 8;
            n -= 8;
        }
        while (n--) c = (c >> 8) ^ t[0][(c ^ *p++) & 0xFF];
        return ~c;
    }
};
const Crc32c &crc_table() {
    static const Crc32c tab;
    return tab;
}
uint32_t crc32c(uint32_t crc, const void *p, size_t n) { return crc_table()(crc, (const uint8_t *)p, n); }

/* ---- SHA-256 (FIPS 180-4) ------------------------------------------------- */
struct Sha256 {
    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
    static void block(uint32_t h[8], const uint8_t *p) {
        static const uint32_t K[64] = {
            0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
            0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
            0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
            0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
            0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
            0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
            0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
            0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
        uint32_t w[64];
        for (int i = 0; i < 16; i++)
            w[i] = ((uint32_t)p[4 * i] << 24) | ((uint32_t)p[4 * i + 1] << 16) | ((uint32_t)p[4 * i + 2] << 8) |
                   p[4 * i + 3];
        for (int i = 16; i < 64; i++) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], k = h[7];
        for (int i = 0; i < 64; i++) {
            const uint32_t t1 = k + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + K[i] + w[i];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            k = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = b;
            b = a;
            a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += k;
    }
    static void digest(const uint8_t *p, size_t n, uint8_t out[32]) {
        uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab,
                         0x5be0cd19};
        size_t i = 0;
        for (; i + 64 <= n; i += 64) block(h, p + i);
        uint8_t tail[128] = {};
        const size_t r = n - i;
        memcpy(tail, p + i, r);
        tail[r] = 0x80;
        const size_t tl = r + 9 <= 64 ? 64 : 128;
        const uint64_t bits = (uint64_t)n * 8;
        for (int b = 0; b < 8; b++) tail[tl - 1 - b] = (uint8_t)(bits >> (8 * b));
        block(h, tail);
        if (tl == 128) block(h, tail + 64);
        for (int j = 0; j < 8; j++)
            for (int b = 0; b < 4; b++) out[4 * j + b] = (uint8_t)(h[j] >> (24 - 8 * b));
    }
};

bool str_ok(const char *s, size_t cap, bool allow_empty) { return memchr(s, 0, cap) && (allow_empty || s[0]); }

/* ---- packet table rules ------------------------------------------------------
 * What a loaded table must satisfy (the format of src/lib/tlm_packet.h:39-95,
 * the same rejections as the reference's loader, src/lib/tlm_packet.c:
 * 211-275): each record is checked against the list of per-record rules
 * below, the table must be in strictly increasing (type, layer, id) order,
 * and no two byte ranges (a packet or its replica) may share bytes of one
 * drive file. */
using PacketKey = std::tuple<uint16_t, uint16_t, uint32_t>;
PacketKey packet_key(const tlm_hip_packet_loc &l) { return PacketKey(l.type, l.layer, l.id); }

bool aligned_range(uint64_t off, uint64_t len) { return off % ALIGN_IO == 0 && off <= UINT64_MAX - len; }

struct RecordRule {
    const char *what;
    bool (*ok)(const tlm_hip_packet_loc &, uint32_t n_drives);
};
const RecordRule RECORD_RULES[] = {
    {"type outside DENSE..TOKEN",
     [](const tlm_hip_packet_loc &l, uint32_t) { return l.type >= TLM_HIP_PK_DENSE && l.type <= TLM_HIP_PK_TOKEN; }},
    {"drive index past the drive list", [](const tlm_hip_packet_loc &l, uint32_t nd) { return l.drive < nd; }},
    {"replica drive invalid or equal to the primary",
     [](const tlm_hip_packet_loc &l, uint32_t nd) {
         return l.replica_drive == 0xFF || (l.replica_drive < nd && l.replica_drive != l.drive);
     }},
    {"flag bits this format does not define",
     [](const tlm_hip_packet_loc &l, uint32_t) { return (l.flags & ~KNOWN_FLAGS) == 0; }},
    {"length not a positive multiple of 4096 within the payload limit",
     [](const tlm_hip_packet_loc &l, uint32_t) {
         return l.total_len >= ALIGN_IO && l.total_len % ALIGN_IO == 0 && l.total_len <= MAX_PAYLOAD + ALIGN_IO;
     }},
    {"offset not 4096-aligned or wrapping", [](const tlm_hip_packet_loc &l, uint32_t) { return aligned_range(l.offset, l.total_len); }},
    {"replica offset not 4096-aligned or wrapping",
     [](const tlm_hip_packet_loc &l, uint32_t) {
         return l.replica_drive == 0xFF || aligned_range(l.replica_offset, l.total_len);
     }},
    {"heat negative or not finite", [](const tlm_hip_packet_loc &l, uint32_t) { return std::isfinite(l.heat) && l.heat >= 0.0f; }},
};

int check_table(const std::vector<tlm_hip_packet_loc> &p, uint32_t n_drives) {
    /* byte ranges per drive: [first, last) with the record that owns them */
    std::vector<std::vector<std::pair<uint64_t, uint32_t>>> starts(n_drives);
    for (uint32_t i = 0; i < (uint32_t)p.size(); i++) {
        const tlm_hip_packet_loc &l = p[i];
        for (const RecordRule &r : RECORD_RULES)
            if (!r.ok(l, n_drives))
                return tlmh_seterr(TLM_HIP_EFORMAT, "store table: record %u (type %u, layer %u, id %u): %s", i, l.type,
                                   l.layer, l.id, r.what);
        if (i && !(packet_key(p[i - 1]) < packet_key(l)))
            return tlmh_seterr(TLM_HIP_EFORMAT, "store table: record %u is not after record %u in (type, layer, id) "
                               "order", i, i - 1);
        starts[l.drive].push_back({l.offset, i});
        if (l.replica_drive != 0xFF) starts[l.replica_drive].push_back({l.replica_offset, i});
    }
    for (uint32_t d = 0; d < n_drives; d++) {
        auto &v = starts[d];
        std::sort(v.begin(), v.end());
        for (size_t j = 1; j < v.size(); j++)
            if (v[j - 1].first + p[v[j - 1].second].total_len > v[j].first)
                return tlmh_seterr(TLM_HIP_EFORMAT, "store table: records %u and %u claim the same bytes of drive %u",
                                   v[j - 1].second, v[j].second, d);
    }
    return TLM_HIP_OK;
}

int read_file(const char *path, std::vector<uint8_t> &out) {
    FILE *f = fopen(path, "rb");
    if (!f) return tlmh_seterr(TLM_HIP_EIO, "cannot open %s", path);
    if (fseek(f, 0, SEEK_END) != 0) {
        fclose(f);
        return tlmh_seterr(TLM_HIP_EIO, "cannot size %s", path);
    }
    const long n = ftell(f);
    if (n < 0 || fseek(f, 0, SEEK_SET) != 0) {
        fclose(f);
        return tlmh_seterr(TLM_HIP_EIO, "cannot size %s", path);
    }
    out.resize((size_t)n);
    const size_t got = n ? fread(out.data(), 1, (size_t)n, f) : 0;
    fclose(f);
    if (got != (size_t)n) return tlmh_seterr(TLM_HIP_EIO, "short read of %s", path);
    return TLM_HIP_OK;
}

}  // namespace

struct tlm_hip_manifest {
    tlm_hip_model_geom geom{};
    char name[64] = {}, profile[16] = {};
    std::vector<std::string> drives;      /* packet file per drive */
    std::vector<tlm_hip_packet_loc> packets;
    uint32_t n_pruned = 0;
    uint8_t table_sha256[32] = {}, source_sha256[32] = {};
    std::vector<int> fd;                  /* opened lazily, one per drive */
    ~tlm_hip_manifest() {
        for (int f : fd)
            if (f >= 0) close(f);
    }
};

extern "C" {

/* ---- the manifest file ----------------------------------------------------------
 * Layout (src/lib/tlm_packet.h:39-95, src/lib/tlm_packet.c:8-34): a 512-byte
 * fixed header, the drive paths (256 bytes each), the packet table (48-byte
 * records) and a text report, back to back, with the header's own CRC32C over
 * its first 508 bytes and the drive paths, the table's SHA-256 and the
 * report's CRC32C.  The header's section fields are checked as a list of rules
 * on the decoded values, then the checksums, then the strings and records. */
struct ManifestHeader {
    uint32_t magic, version, fixed, rec, n_drives, n_packets, n_pruned, report_crc, header_crc;
    uint64_t drives_off, table_off, table_len, report_off, report_len, file_size, actual;
    explicit ManifestHeader(const uint8_t *b, size_t size)
        : magic(rd32(b)), version(rd32(b + 4)), fixed(rd32(b + 8)), rec(rd32(b + 12)), n_drives(rd32(b + 16)),
          n_packets(rd32(b + 20)), n_pruned(rd32(b + 24)), report_crc(rd32(b + 28)), header_crc(rd32(b + CRC_AT)),
          drives_off(rd64(b + 32)), table_off(rd64(b + 40)), table_len(rd64(b + 48)), report_off(rd64(b + 56)),
          report_len(rd64(b + 64)), file_size(rd64(b + 72)), actual(size) {}
};

struct HeaderRule {
    const char *what;
    bool (*ok)(const ManifestHeader &);
};
const HeaderRule HEADER_RULES[] = {
    {"not a tierlm manifest (magic)", [](const ManifestHeader &h) { return h.magic == MANIFEST_MAGIC; }},
    {"store format version other than 2", [](const ManifestHeader &h) { return h.version == STORE_VERSION; }},
    {"header or record size not 512 / 48", [](const ManifestHeader &h) { return h.fixed == FIXED && h.rec == REC_BYTES; }},
    {"drive count outside 1..16", [](const ManifestHeader &h) { return h.n_drives >= 1 && h.n_drives <= MAX_DRIVES; }},
    {"more than 2^24 packets", [](const ManifestHeader &h) { return h.n_packets <= MAX_PACKETS; }},
    {"more pruned packets than packets", [](const ManifestHeader &h) { return h.n_pruned <= h.n_packets; }},
    {"drive list not right after the header", [](const ManifestHeader &h) { return h.drives_off == FIXED; }},
    {"packet table not right after the drive list",
     [](const ManifestHeader &h) { return h.table_off == h.drives_off + (uint64_t)h.n_drives * DRIVE_BYTES; }},
    {"packet table length not 48 bytes per packet",
     [](const ManifestHeader &h) { return h.table_len == (uint64_t)h.n_packets * REC_BYTES; }},
    {"report not right after the packet table",
     [](const ManifestHeader &h) { return h.report_off == h.table_off + h.table_len; }},
    {"report longer than 64 MiB", [](const ManifestHeader &h) { return h.report_len <= MAX_REPORT; }},
    {"recorded file size disagrees with the sections or the file",
     [](const ManifestHeader &h) { return h.file_size == h.report_off + h.report_len && h.file_size == h.actual; }},
};

int tlm_hip_manifest_load(const char *path, tlm_hip_manifest **out) {
    if (!path || !out) return tlmh_seterr(TLM_HIP_EINVAL, "manifest load: NULL argument");
    *out = nullptr;
    std::vector<uint8_t> raw;
    if (int rc = read_file(path, raw)) return rc;
    const uint8_t *b = raw.data();
    if (raw.size() < FIXED)
        return tlmh_seterr(TLM_HIP_EFORMAT, "%s: %zu bytes, shorter than a manifest header", path, raw.size());
    const ManifestHeader h(b, raw.size());
    for (const HeaderRule &r : HEADER_RULES)
        if (!r.ok(h)) return tlmh_seterr(TLM_HIP_EFORMAT, "%s: %s", path, r.what);

    /* integrity: header CRC32C (first 508 bytes, then the drive paths), table
     * SHA-256 (stored at byte 80), report CRC32C and its text */
    if (crc32c(crc32c(0, b, CRC_AT), b + FIXED, (size_t)h.n_drives * DRIVE_BYTES) != h.header_crc)
        return tlmh_seterr(TLM_HIP_EFORMAT, "%s: header CRC32C does not match its contents", path);
    uint8_t sha[32];
    Sha256::digest(b + h.table_off, (size_t)h.table_len, sha);
    if (memcmp(sha, b + 80, 32) != 0)
        return tlmh_seterr(TLM_HIP_EFORMAT, "%s: packet table does not hash to the recorded SHA-256", path);
    if ((h.report_len ? crc32c(0, b + h.report_off, (size_t)h.report_len) : 0u) != h.report_crc)
        return tlmh_seterr(TLM_HIP_EFORMAT, "%s: report CRC32C does not match its text", path);
    if (h.report_len && memchr(b + h.report_off, 0, (size_t)h.report_len))
        return tlmh_seterr(TLM_HIP_EFORMAT, "%s: report text holds a NUL byte", path);

    std::unique_ptr<tlm_hip_manifest> m(new tlm_hip_manifest);
    memcpy(m->table_sha256, b + 80, 32);
    memcpy(m->source_sha256, b + 112, 32);
    memcpy(m->name, b + 176, 64);
    memcpy(m->profile, b + 240, 16);
    /* geometry (src/lib/tlm_packet.c:535-548): the architecture string, then
     * u32 / f32 fields in this order */
    tlm_hip_model_geom &g = m->geom;
    memcpy(g.arch, b + 256, 32);
    struct Field {
        uint32_t *u;
        float *f;
    };
    const Field geom_fields[] = {
        {&g.n_layers, nullptr}, {&g.d_model, nullptr}, {&g.n_heads, nullptr}, {&g.n_kv_heads, nullptr},
        {&g.head_dim, nullptr}, {&g.vocab, nullptr}, {&g.n_experts, nullptr}, {&g.top_k, nullptr},
        {&g.d_expert, nullptr}, {&g.n_shared, nullptr}, {&g.d_shared, nullptr}, {&g.max_ctx, nullptr},
        {&g.router, nullptr}, {nullptr, &g.rope_theta}, {nullptr, &g.norm_eps}, {nullptr, &g.routed_scale},
        {&g.mtp_layers, nullptr}, {&g.rope_scale, nullptr}, {nullptr, &g.rope_factor}, {nullptr, &g.rope_beta_fast},
        {nullptr, &g.rope_beta_slow}, {&g.rope_orig_len, nullptr}};
    const uint8_t *gp = b + 288;
    for (const Field &f : geom_fields) {
        if (f.u) *f.u = rd32(gp);
        else *f.f = rdf(gp);
        gp += 4;
    }
    const bool name_ok = str_ok(m->name, 64, false) && !strchr(m->name, '/') && strcmp(m->name, ".") != 0 &&
                         strcmp(m->name, "..") != 0;
    if (!name_ok || !str_ok(m->profile, 16, true) || !str_ok(g.arch, 32, true))
        return tlmh_seterr(TLM_HIP_EFORMAT, "%s: store name, profile or architecture is not a terminated string "
                           "(or the name is a path)", path);
    for (uint32_t i = 0; i < h.n_drives; i++) {
        const char *dir = (const char *)(b + h.drives_off + (size_t)i * DRIVE_BYTES);
        if (!str_ok(dir, DRIVE_BYTES, false))
            return tlmh_seterr(TLM_HIP_EFORMAT, "%s: drive %u path is empty or unterminated", path, i);
        m->drives.push_back(std::string(dir) + "/" + m->name + ".tlmp");   /* tlm_packet.c:780-786 */
    }
    m->fd.assign(h.n_drives, -1);
    m->n_pruned = h.n_pruned;
    /* records (src/lib/tlm_packet.c:565-578): type u16, layer u16, id u32,
     * drive u8, replica drive u8, flags u16, crc32c u32, offset u64, replica
     * offset u64, total length u64, heat f32, 4 bytes spare */
    m->packets.resize(h.n_packets);
    for (uint32_t i = 0; i < h.n_packets; i++) {
        const uint8_t *r = b + h.table_off + (size_t)i * REC_BYTES;
        m->packets[i] = tlm_hip_packet_loc{};
        tlm_hip_packet_loc &l = m->packets[i];
        l.type = rd16(r);
        l.layer = rd16(r + 2);
        l.id = rd32(r + 4);
        l.drive = r[8];
        l.replica_drive = r[9];
        l.flags = rd16(r + 10);
        l.crc32c = rd32(r + 12);
        l.offset = rd64(r + 16);
        l.replica_offset = rd64(r + 24);
        l.total_len = rd64(r + 32);
        l.heat = rdf(r + 40);
    }
    if (int rc = check_table(m->packets, h.n_drives)) return rc;
    *out = m.release();
    return TLM_HIP_OK;
}

void tlm_hip_manifest_free(tlm_hip_manifest *m) { delete m; }

const tlm_hip_model_geom *tlm_hip_manifest_geom(const tlm_hip_manifest *m) { return m ? &m->geom : nullptr; }
const char *tlm_hip_manifest_name(const tlm_hip_manifest *m) { return m ? m->name : nullptr; }
int tlm_hip_manifest_n_packets(const tlm_hip_manifest *m) { return m ? (int)m->packets.size() : 0; }

const tlm_hip_packet_loc *tlm_hip_manifest_packet(const tlm_hip_manifest *m, int i) {
    return m && i >= 0 && i < (int)m->packets.size() ? &m->packets[i] : nullptr;
}

/* src/lib/tlm_packet.c:761-778: binary search of the sorted table */
const tlm_hip_packet_loc *tlm_hip_manifest_find(const tlm_hip_manifest *m, int type, int layer, uint32_t id) {
    if (!m) return nullptr;
    tlm_hip_packet_loc key{};
    key.type = (uint16_t)type;
    key.layer = (uint16_t)layer;
    key.id = id;
    auto it = std::lower_bound(m->packets.begin(), m->packets.end(), key,
                               [](const tlm_hip_packet_loc &a, const tlm_hip_packet_loc &b) {
                                   return packet_key(a) < packet_key(b);
                               });
    return it != m->packets.end() && packet_key(*it) == packet_key(key) ? &*it : nullptr;
}

const char *tlm_hip_manifest_drive_path(const tlm_hip_manifest *m, int i) {
    return m && i >= 0 && i < (int)m->drives.size() ? m->drives[i].c_str() : nullptr;
}

/* src/lib/tlm_packet.c:788-832: read loc->total_len bytes into buf, check the
 * header against the record, the length, and the payload CRC; on a bad
 * primary copy the replica is read and checked the same way. */
int tlm_hip_packet_read(tlm_hip_manifest *m, const tlm_hip_packet_loc *loc, void *buf, uint64_t *payload_off,
                        uint64_t *payload_len) {
    if (!m || !loc || !buf) return tlmh_seterr(TLM_HIP_EINVAL, "packet read: missing manifest, record or buffer");
    int rc = TLM_HIP_EIO;
    for (int copy = 0; copy < 2 && rc; copy++) {
        const int drive = copy == 0 ? loc->drive : loc->replica_drive;
        if (copy == 1 && loc->replica_drive == 0xFF) break;
        const uint64_t off = copy == 0 ? loc->offset : loc->replica_offset;
        if (m->fd[drive] < 0) m->fd[drive] = open(m->drives[drive].c_str(), O_RDONLY | O_CLOEXEC);
        if (m->fd[drive] < 0) {
            rc = tlmh_seterr(TLM_HIP_EIO, "cannot open %s", m->drives[drive].c_str());
            continue;
        }
        uint64_t got = 0;
        while (got < loc->total_len) {
            const ssize_t r = pread(m->fd[drive], (uint8_t *)buf + got, (size_t)(loc->total_len - got), (off_t)(off + got));
            if (r <= 0) break;
            got += (uint64_t)r;
        }
        if (got != loc->total_len) {
            rc = tlmh_seterr(TLM_HIP_EIO, "%s: file ends inside packet (%u, %u, %u)", m->drives[drive].c_str(), loc->type, loc->layer, loc->id);
            continue;
        }
        const uint8_t *h = (const uint8_t *)buf;   /* tlm_packet_hdr, tlm_packet.h:39-54 */
        const uint64_t plen = rd64(h + 24);
        if (rd32(h) != PACKET_MAGIC || rd16(h + 6) != STORE_VERSION)
            rc = tlmh_seterr(TLM_HIP_EFORMAT, "packet (%u, %u, %u): not a packet of this store version", loc->type,
                             loc->layer, loc->id);
        else if (rd16(h + 4) != loc->type || rd16(h + 8) != loc->layer || rd32(h + 12) != loc->id)
            rc = tlmh_seterr(TLM_HIP_EFORMAT, "packet (%u, %u, %u): its header names another packet than the manifest record",
                             loc->type, loc->layer, loc->id);
        else if (plen > loc->total_len - HDR_BYTES || (HDR_BYTES + plen + ALIGN_IO - 1) / ALIGN_IO * ALIGN_IO != loc->total_len)
            rc = tlmh_seterr(TLM_HIP_EFORMAT, "packet (%u, %u, %u): payload length disagrees with the record", loc->type,
                             loc->layer, loc->id);
        else {
            const uint32_t c = plen ? crc32c(0, h + HDR_BYTES, (size_t)plen) : 0;
            if (c != rd32(h + 32) || c != loc->crc32c)
                rc = tlmh_seterr(TLM_HIP_EFORMAT, "packet (%u, %u, %u): payload CRC32C check failed", loc->type,
                                 loc->layer, loc->id);
            else {
                rc = TLM_HIP_OK;
                if (payload_off) *payload_off = HDR_BYTES;
                if (payload_len) *payload_len = plen;
            }
        }
    }
    return rc;
}

/* The item offsets and dtype of an EXPERT packet's header (tlm_packet.h:39-54). */
int tlm_hip_packet_header(const void *buf, uint32_t *dtype, uint32_t item_off[3]) {
    if (!buf) return tlmh_seterr(TLM_HIP_EINVAL, "packet header: NULL");
    const uint8_t *h = (const uint8_t *)buf;
    if (dtype) *dtype = rd32(h + 16);
    if (item_off)
        for (int i = 0; i < 3; i++) item_off[i] = rd32(h + 36 + 4 * i);
    return TLM_HIP_OK;
}

/* Tensor directory lookup (tlm_packet.c:877-917): the entry named `name` of a
 * DENSE / META / EMBED payload, bounds-checked; TLM_HIP_ENOTFOUND if absent. */
int tlm_hip_dir_find(const void *payload, uint64_t len, const char *name, tlm_hip_tensor_ref *out) {
    if (!payload || !name || !out) return tlmh_seterr(TLM_HIP_EINVAL, "dir find: missing payload, name or output");
    const uint8_t *p = (const uint8_t *)payload;
    if (len < 8) return tlmh_seterr(TLM_HIP_EFORMAT, "tensor directory: payload shorter than its header");
    const uint32_t n = rd32(p);
    constexpr uint64_t REF = 88;   /* tlm_tensor_ref, packed */
    if ((uint64_t)n * REF > len - 8) return tlmh_seterr(TLM_HIP_EFORMAT, "tensor directory: %u records do not fit the payload", n);
    const uint64_t data_start = 8 + (uint64_t)n * REF;
    for (uint32_t i = 0; i < n; i++) {
        const uint8_t *r = p + 8 + (size_t)i * REF;
        tlm_hip_tensor_ref t{};
        memcpy(t.name, r, 48);
        t.dtype = rd32(r + 48);
        t.ndim = rd32(r + 52);
        t.shape[0] = rd64(r + 56);
        t.shape[1] = rd64(r + 64);
        t.offset = rd64(r + 72);
        t.nbytes = rd64(r + 80);
        const bool ok = memchr(t.name, 0, 48) && t.name[0] && (t.ndim == 1 || t.ndim == 2) &&
                        t.offset % ALIGN_DIR == 0 && t.offset <= len && t.nbytes <= len - t.offset &&
                        t.offset >= data_start;
        if (!ok) return tlmh_seterr(TLM_HIP_EFORMAT, "tensor directory: record %u lies outside the payload", i);
        if (strncmp(t.name, name, 48) == 0) {
            *out = t;
            return TLM_HIP_OK;
        }
    }
    return TLM_HIP_ENOTFOUND;
}

/* CRC32C and SHA-256 as used by the format, for callers that check files. */
uint32_t tlm_hip_crc32c(uint32_t crc, const void *p, size_t n) { return crc32c(crc, p, n); }
void tlm_hip_sha256(const void *p, size_t n, uint8_t out[32]) { Sha256::digest((const uint8_t *)p, n, out); }

}  // extern "C"
