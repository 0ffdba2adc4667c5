/* sp_hash.c -- the three published hash functions the .sp-model format uses,
 * written from their specifications:
 *   CRC-32   ISO-HDLC / zlib: reflected polynomial 0xEDB88320, init and final
 *            xor 0xFFFFFFFF (include/sp/sp_hash.h:28-31; KAT "123456789" -> 0xCBF43926)
 *   SHA-256  FIPS 180-4
 *   XXH64    xxHash 64-bit, Y. Collet's published algorithm
 * plus the format's 32-byte per-tensor digest field, which the reference fills
 * with SHA-256 over a 16-byte tag followed by the data (core/io_hash/sp_hash.c:157-163);
 * only the byte values of the tag are reproduced so that written files match. */
#include "sp_model_abi.h"
#include <string.h>

/* ---------------- CRC-32 ---------------- */
static uint32_t crc_tab[256];
static int crc_ready;
static void crc_init(void) {
    for (uint32_t i = 0; i < 256; i++) {
        uint32_t c = i;
        for (int k = 0; k < 8; k++) c = (c >> 1) ^ (0xEDB88320u & (0u - (c & 1u)));
        crc_tab[i] = c;
    }
    crc_ready = 1;
}
uint32_t sp_crc32(const void *data, size_t len) {
    if (!crc_ready) crc_init();
    const uint8_t *p = (const uint8_t *)data;
    uint32_t c = 0xFFFFFFFFu;
    for (size_t i = 0; i < len; i++) c = crc_tab[(c ^ p[i]) & 255u] ^ (c >> 8);
    return c ^ 0xFFFFFFFFu;
}

/* ---------------- SHA-256 ---------------- */
typedef struct { uint32_t h[8]; uint64_t nbytes; uint8_t blk[64]; size_t fill; } sha_ctx;
static const uint32_t SHA_K[64] = {
    0x428a2f98,0x71374491,0xb5c0fbcf,0xe9b5dba5,0x3956c25b,0x59f111f1,0x923f82a4,0xab1c5ed5,
    0xd807aa98,0x12835b01,0x243185be,0x550c7dc3,0x72be5d74,0x80deb1fe,0x9bdc06a7,0xc19bf174,
    0xe49b69c1,0xefbe4786,0x0fc19dc6,0x240ca1cc,0x2de92c6f,0x4a7484aa,0x5cb0a9dc,0x76f988da,
    0x983e5152,0xa831c66d,0xb00327c8,0xbf597fc7,0xc6e00bf3,0xd5a79147,0x06ca6351,0x14292967,
    0x27b70a85,0x2e1b2138,0x4d2c6dfc,0x53380d13,0x650a7354,0x766a0abb,0x81c2c92e,0x92722c85,
    0xa2bfe8a1,0xa81a664b,0xc24b8b70,0xc76c51a3,0xd192e819,0xd6990624,0xf40e3585,0x106aa070,
    0x19a4c116,0x1e376c08,0x2748774c,0x34b0bcb5,0x391c0cb3,0x4ed8aa4a,0x5b9cca4f,0x682e6ff3,
    0x748f82ee,0x78a5636f,0x84c87814,0x8cc70208,0x90befffa,0xa4506ceb,0xbef9a3f7,0xc67178f2};
static uint32_t ror(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
static void sha_block(sha_ctx *c, const uint8_t *b) {
    uint32_t w[64];
    for (int i = 0; i < 16; i++)
        w[i] = (uint32_t)b[4*i] << 24 | (uint32_t)b[4*i+1] << 16 | (uint32_t)b[4*i+2] << 8 | b[4*i+3];
    for (int i = 16; i < 64; i++) {
        uint32_t s0 = ror(w[i-15], 7) ^ ror(w[i-15], 18) ^ (w[i-15] >> 3);
        uint32_t s1 = ror(w[i-2], 17) ^ ror(w[i-2], 19) ^ (w[i-2] >> 10);
        w[i] = w[i-16] + s0 + w[i-7] + s1;
    }
    uint32_t v[8];
    memcpy(v, c->h, sizeof v);
    for (int i = 0; i < 64; i++) {
        uint32_t S1 = ror(v[4], 6) ^ ror(v[4], 11) ^ ror(v[4], 25);
        uint32_t ch = (v[4] & v[5]) ^ (~v[4] & v[6]);
        uint32_t t1 = v[7] + S1 + ch + SHA_K[i] + w[i];
        uint32_t S0 = ror(v[0], 2) ^ ror(v[0], 13) ^ ror(v[0], 22);
        uint32_t mj = (v[0] & v[1]) ^ (v[0] & v[2]) ^ (v[1] & v[2]);
        memmove(v + 1, v, 7 * sizeof(uint32_t));
        v[4] += t1;
        v[0] = t1 + S0 + mj;
    }
    for (int i = 0; i < 8; i++) c->h[i] += v[i];
}
static void sha_init(sha_ctx *c) {
    static const uint32_t h0[8] = {0x6a09e667,0xbb67ae85,0x3c6ef372,0xa54ff53a,
                                   0x510e527f,0x9b05688c,0x1f83d9ab,0x5be0cd19};
    memcpy(c->h, h0, sizeof h0); c->nbytes = 0; c->fill = 0;
}
static void sha_update(sha_ctx *c, const void *data, size_t len) {
    const uint8_t *p = (const uint8_t *)data;
    c->nbytes += len;
    while (len) {
        size_t k = 64 - c->fill; if (k > len) k = len;
        memcpy(c->blk + c->fill, p, k); c->fill += k; p += k; len -= k;
        if (c->fill == 64) { sha_block(c, c->blk); c->fill = 0; }
    }
}
static void sha_final(sha_ctx *c, uint8_t out[32]) {
    uint64_t bits = c->nbytes * 8u;
    uint8_t pad = 0x80; sha_update(c, &pad, 1);
    uint8_t z = 0; while (c->fill != 56) sha_update(c, &z, 1);
    uint8_t L[8]; for (int i = 0; i < 8; i++) L[i] = (uint8_t)(bits >> (56 - 8 * i));
    sha_update(c, L, 8);
    for (int i = 0; i < 8; i++) {
        out[4*i] = (uint8_t)(c->h[i] >> 24); out[4*i+1] = (uint8_t)(c->h[i] >> 16);
        out[4*i+2] = (uint8_t)(c->h[i] >> 8); out[4*i+3] = (uint8_t)c->h[i];
    }
}
void sp_sha256(const void *data, size_t len, uint8_t out[32]) {
    sha_ctx c; sha_init(&c); sha_update(&c, data, len); sha_final(&c, out);
}
void sp_blake3_256(const void *data, size_t len, uint8_t out[32]) {
    static const uint8_t tag[16] = {'S','P','-','B','L','A','K','E','3','-','v','0','p','l',0,0};
    sha_ctx c; sha_init(&c); sha_update(&c, tag, sizeof tag); sha_update(&c, data, len);
    sha_final(&c, out);
}

/* ---------------- XXH64 ---------------- */
#define XP1 0x9E3779B185EBCA87ull
#define XP2 0xC2B2AE3D27D4EB4Full
#define XP3 0x165667B19E3779F9ull
#define XP4 0x85EBCA77C2B2AE63ull
#define XP5 0x27D4EB2F165667C5ull
static uint64_t rol64(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
static uint64_t rd64(const uint8_t *p) { uint64_t v; memcpy(&v, p, 8); return v; }
static uint32_t rd32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
static uint64_t xround(uint64_t acc, uint64_t in) { acc += in * XP2; acc = rol64(acc, 31); return acc * XP1; }
static uint64_t xmerge(uint64_t acc, uint64_t v) { acc ^= xround(0, v); return acc * XP1 + XP4; }
uint64_t sp_xxh64(const void *data, size_t len, uint64_t seed) {
    const uint8_t *p = (const uint8_t *)data, *end = p + len;
    uint64_t h;
    if (len >= 32) {
        uint64_t a = seed + XP1 + XP2, b = seed + XP2, c = seed, d = seed - XP1;
        const uint8_t *lim = end - 32;
        do {
            a = xround(a, rd64(p)); b = xround(b, rd64(p + 8));
            c = xround(c, rd64(p + 16)); d = xround(d, rd64(p + 24)); p += 32;
        } while (p <= lim);
        h = rol64(a, 1) + rol64(b, 7) + rol64(c, 12) + rol64(d, 18);
        h = xmerge(h, a); h = xmerge(h, b); h = xmerge(h, c); h = xmerge(h, d);
    } else {
        h = seed + XP5;
    }
    h += (uint64_t)len;
    while (p + 8 <= end) { h ^= xround(0, rd64(p)); h = rol64(h, 27) * XP1 + XP4; p += 8; }
    if (p + 4 <= end) { h ^= (uint64_t)rd32(p) * XP1; h = rol64(h, 23) * XP2 + XP3; p += 4; }
    while (p < end) { h ^= (uint64_t)(*p) * XP5; h = rol64(h, 11) * XP1; p++; }
    h ^= h >> 33; h *= XP2; h ^= h >> 29; h *= XP3; h ^= h >> 32;
    return h;
}
