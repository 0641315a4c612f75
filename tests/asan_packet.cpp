/* asan_packet.cpp - the store reader (tierlm_amd/csrc/host_packet.cpp) under
 * AddressSanitizer and UndefinedBehaviorSanitizer on the CPU, fed a compiled
 * store and damaged copies of it.  Built and run by tests/test_packet_asan.py:
 *
 *   g++ -fsanitize=address,undefined ... asan_packet.cpp host_packet.cpp
 *   asan_packet STORE.tlmm WORKDIR
 *
 * Every manifest variant below must load or be refused with an error code,
 * and every packet / tensor directory must read or be refused, without a
 * sanitizer report (the sanitizers abort the process on the first one).
 * Variants: every byte of the header and drive list flipped; truncations;
 * packet records rewritten with hostile values and the table's SHA-256 and
 * header CRC recomputed, so the record checks run on them; every packet of
 * the store read and its tensor directory searched; directories with bytes
 * flipped and lengths cut short. */
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "../include/tlm_hip.h"

static char g_msg[512];
int tlmh_seterr(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof g_msg, fmt, ap);
    va_end(ap);
    return code;
}

static std::vector<uint8_t> slurp(const char *path) {
    std::vector<uint8_t> v;
    FILE *f = fopen(path, "rb");
    if (!f) return v;
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    v.resize((size_t)n);
    if (fread(v.data(), 1, v.size(), f) != v.size()) v.clear();
    fclose(f);
    return v;
}

static void spill(const std::string &path, const std::vector<uint8_t> &v) {
    FILE *f = fopen(path.c_str(), "wb");
    if (!v.empty()) fwrite(v.data(), 1, v.size(), f);
    fclose(f);
}

static uint32_t rd32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
static uint64_t rd64(const uint8_t *p) { uint64_t v; memcpy(&v, p, 8); return v; }

/* re-seal a manifest image after its records changed: table SHA-256 at byte
 * 80, then the header CRC32C (first 508 bytes + the drive list) */
static void reseal(std::vector<uint8_t> &m) {
    const uint32_t nd = rd32(&m[16]);
    const uint64_t toff = rd64(&m[40]), tlen = rd64(&m[48]);
    if (toff <= m.size() && tlen <= m.size() - toff) tlm_hip_sha256(&m[toff], (size_t)tlen, &m[80]);
    if (nd > (m.size() - 512) / 256) return;   /* a drive count past the file: left unsealed */
    uint32_t c = tlm_hip_crc32c(0, m.data(), 508);
    c = tlm_hip_crc32c(c, &m[512], (size_t)nd * 256);
    memcpy(&m[508], &c, 4);
}

static int try_load(const std::string &path, const std::vector<uint8_t> &img, int *ok) {
    spill(path, img);
    tlm_hip_manifest *m = nullptr;
    const int rc = tlm_hip_manifest_load(path.c_str(), &m);
    if (rc == 0) {
        (*ok)++;
        for (int i = 0; i < tlm_hip_manifest_n_packets(m); i++) {
            const tlm_hip_packet_loc *l = tlm_hip_manifest_packet(m, i);
            if (i < 12 && l->total_len <= (1u << 20)) {   /* read the records the variants rewrite */
                std::vector<uint8_t> buf(l->total_len);
                uint64_t off = 0, len = 0;
                if (tlm_hip_packet_read(m, l, buf.data(), &off, &len) == 0 && l->type != TLM_HIP_PK_EXPERT) {
                    tlm_hip_tensor_ref t;
                    (void)tlm_hip_dir_find(buf.data() + off, len, "attn_q", &t);
                }
            }
        }
        (void)tlm_hip_manifest_find(m, 1, 0, 0);
        tlm_hip_manifest_free(m);
    } else if (rc > 0) {
        fprintf(stderr, "positive return code %d\n", rc);
        exit(3);
    }
    return rc;
}

static void dir_probe(const uint8_t *payload, uint64_t len) {
    static const char *names[] = {"attn_q", "attn_k", "attn_norm", "router", "lm_head", "tok_embd", "output_norm",
                                  "shared_gate", "no_such_tensor"};
    for (const char *n : names) {
        tlm_hip_tensor_ref t;
        (void)tlm_hip_dir_find(payload, len, n, &t);
    }
}

int main(int argc, char **argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: asan_packet STORE.tlmm WORKDIR\n");
        return 2;
    }
    const std::vector<uint8_t> base = slurp(argv[1]);
    if (base.size() < 1024) {
        fprintf(stderr, "cannot read %s\n", argv[1]);
        return 2;
    }
    const std::string tmp = std::string(argv[2]) + "/m.tlmm";
    int loaded = 0, refused = 0;

    /* the store itself: every packet read, every directory searched */
    tlm_hip_manifest *m = nullptr;
    if (tlm_hip_manifest_load(argv[1], &m) != 0) {
        fprintf(stderr, "store does not load: %s\n", g_msg);
        return 4;
    }
    std::vector<std::vector<uint8_t>> dirs;
    for (int i = 0; i < tlm_hip_manifest_n_packets(m); i++) {
        const tlm_hip_packet_loc *l = tlm_hip_manifest_packet(m, i);
        std::vector<uint8_t> buf(l->total_len);
        uint64_t off = 0, len = 0;
        if (tlm_hip_packet_read(m, l, buf.data(), &off, &len) != 0) {
            fprintf(stderr, "packet %d does not read: %s\n", i, g_msg);
            return 4;
        }
        uint32_t dt, io[3];
        (void)tlm_hip_packet_header(buf.data(), &dt, io);
        if (l->type != TLM_HIP_PK_EXPERT) {
            dir_probe(buf.data() + off, len);
            if (dirs.size() < 3) dirs.emplace_back(buf.begin() + off, buf.begin() + off + len);
        }
    }
    tlm_hip_manifest_free(m);

    /* every byte of the fixed header and the drive list flipped (the header
     * CRC catches most; re-sealed, the section and record rules run) */
    const uint32_t nd = rd32(&base[16]);
    const size_t head = 512 + (size_t)nd * 256;
    for (size_t at = 0; at < head; at++)
        for (int sealed = 0; sealed < 2; sealed++) {
            std::vector<uint8_t> v = base;
            v[at] ^= (uint8_t)(0x5A + at);
            if (sealed) reseal(v);
            if (try_load(tmp, v, &loaded) < 0) refused++;
        }
    /* truncations */
    for (size_t cut : {(size_t)0, (size_t)7, (size_t)511, (size_t)512, head - 1, head + 47, base.size() - 1})
        if (cut < base.size()) try_load(tmp, std::vector<uint8_t>(base.begin(), base.begin() + cut), &loaded);
    /* hostile records, re-sealed */
    const uint64_t toff = rd64(&base[40]);
    const uint32_t np = rd32(&base[20]);
    const uint64_t hostile64[] = {0, 1, 4095, 4096, 1ull << 40, (1ull << 40) + 8192, ~0ull - 4095, ~0ull};
    for (uint32_t r = 0; r < np && r < 12; r++)
        for (int field = 0; field < 7; field++)
            for (uint64_t hv : hostile64) {
                std::vector<uint8_t> v = base;
                uint8_t *rec = &v[toff + (size_t)r * 48];
                switch (field) {
                case 0: rec[0] = (uint8_t)hv; rec[1] = (uint8_t)(hv >> 8); break;     /* type */
                case 1: rec[8] = (uint8_t)hv; break;                                  /* drive */
                case 2: rec[9] = (uint8_t)hv; break;                                  /* replica drive */
                case 3: rec[10] = (uint8_t)hv; rec[11] = (uint8_t)(hv >> 8); break;   /* flags */
                case 4: memcpy(rec + 16, &hv, 8); break;                              /* offset */
                case 5: memcpy(rec + 24, &hv, 8); rec[9] = 0; break;                  /* replica offset */
                case 6: memcpy(rec + 32, &hv, 8); break;                              /* length */
                }
                reseal(v);
                try_load(tmp, v, &loaded);
            }
    /* damaged tensor directories */
    for (const std::vector<uint8_t> &d : dirs) {
        for (size_t at = 0; at < d.size() && at < 4096; at += 3) {
            std::vector<uint8_t> v = d;
            v[at] ^= 0xA5;
            dir_probe(v.data(), v.size());
        }
        for (size_t cut = 0; cut < d.size() && cut < 4096; cut += 61) {
            std::vector<uint8_t> v(d.begin(), d.begin() + cut);
            dir_probe(v.data(), v.size());
        }
    }
    printf("asan_packet: done (%d variants loaded, %d header variants refused)\n", loaded, refused);
    return 0;
}
