// Model and checkpoint files straight from HBM (src/etalii_dllm/modelfile.py:68-136,228-235 and
// training/trainer.py:534-630): SHA-256 fingerprints of the tensor data and the byte layout of model.dllm and
// .dllmckpt files.
//
// The fingerprint is one SHA-256 chain over the tensor data section: float32 bytes of each tensor in order, each
// padded with zero bytes to a multiple of 64. SHA-256 is a serial chain over the message, so it runs on the host.
// The tensors stream out of device memory through two pinned buffers: the copy of the next buffer is in flight while
// the host hashes (and writes) the current one.
//
// File layout (both formats): a prefix (magic, u32 version, u64 header length, little-endian), the header (canonical
// JSON, padded with spaces so the data starts at a multiple of 64), then the data section. The header holds a
// 64-character placeholder fingerprint ("fingerprint":"000...0"), patched in place once the data is hashed.
#include <immintrin.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "common.h"
#include "export.h"

namespace dllm_hip {

namespace {

// ---- SHA-256 (FIPS 180-4) ----

constexpr uint32_t kK[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

void blocks_portable(uint32_t h[8], const uint8_t* p, size_t blocks) {
    for (; blocks > 0; --blocks, p += 64) {
        uint32_t w[64];
        for (int t = 0; t < 16; ++t)
            w[t] = (uint32_t{p[4 * t]} << 24) | (uint32_t{p[4 * t + 1]} << 16) | (uint32_t{p[4 * t + 2]} << 8) |
                   uint32_t{p[4 * t + 3]};
        for (int t = 16; t < 64; ++t) {
            const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
            const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
            w[t] = w[t - 16] + s0 + w[t - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int t = 0; t < 64; ++t) {
            const uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + kK[t] + w[t];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            hh = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = b;
            b = a;
            a = t1 + t2;
        }
        h[0] += a;
        h[1] += b;
        h[2] += c;
        h[3] += d;
        h[4] += e;
        h[5] += f;
        h[6] += g;
        h[7] += hh;
    }
}

// The same compression with the x86 SHA extensions: the state is kept as the register pair (A B E F), (C D G H) that
// sha256rnds2 works on; each sha256rnds2 does two rounds; the schedule is w[t] = msg2(msg1(w[t-16..], w[t-12..]) +
// w[t-7..], w[t-4..]) four words at a time.
__attribute__((target("sha,sse4.1"))) void blocks_shani(uint32_t h[8], const uint8_t* p, size_t blocks) {
    const __m128i swap = _mm_set_epi64x(0x0c0d0e0f08090a0bLL, 0x0405060700010203LL);
    __m128i abcd = _mm_loadu_si128(reinterpret_cast<const __m128i*>(&h[0]));  // lanes: a b c d
    __m128i efgh = _mm_loadu_si128(reinterpret_cast<const __m128i*>(&h[4]));  // lanes: e f g h
    abcd = _mm_shuffle_epi32(abcd, 0xB1);                                      // b a d c
    efgh = _mm_shuffle_epi32(efgh, 0x1B);                                      // h g f e
    __m128i s0 = _mm_alignr_epi8(abcd, efgh, 8);                               // f e b a
    __m128i s1 = _mm_blend_epi16(efgh, abcd, 0xF0);                            // h g d c
    for (; blocks > 0; --blocks, p += 64) {
        const __m128i save0 = s0, save1 = s1;
        __m128i w[4];
        for (int i = 0; i < 4; ++i)
            w[i] = _mm_shuffle_epi8(_mm_loadu_si128(reinterpret_cast<const __m128i*>(p + 16 * i)), swap);
        for (int g = 0; g < 16; ++g) {
            __m128i& cur = w[g & 3];
            if (g >= 4) {
                __m128i t = _mm_sha256msg1_epu32(cur, w[(g + 1) & 3]);  // w[g-4], w[g-3]
                t = _mm_add_epi32(t, _mm_alignr_epi8(w[(g + 3) & 3], w[(g + 2) & 3], 4));  // + w[t-7..t-4]
                cur = _mm_sha256msg2_epu32(t, w[(g + 3) & 3]);
            }
            __m128i m = _mm_add_epi32(cur, _mm_loadu_si128(reinterpret_cast<const __m128i*>(&kK[4 * g])));
            s1 = _mm_sha256rnds2_epu32(s1, s0, m);
            m = _mm_shuffle_epi32(m, 0x0E);
            s0 = _mm_sha256rnds2_epu32(s0, s1, m);
        }
        s0 = _mm_add_epi32(s0, save0);
        s1 = _mm_add_epi32(s1, save1);
    }
    const __m128i feba = _mm_shuffle_epi32(s0, 0x1B);
    const __m128i dchg = _mm_shuffle_epi32(s1, 0xB1);
    const __m128i dcba = _mm_blend_epi16(feba, dchg, 0xF0);
    const __m128i hgfe = _mm_alignr_epi8(dchg, feba, 8);
    _mm_storeu_si128(reinterpret_cast<__m128i*>(&h[0]), dcba);
    _mm_storeu_si128(reinterpret_cast<__m128i*>(&h[4]), hgfe);
}

bool cpu_has_shani() {
    unsigned a = 0, b = 0, c = 0, d = 0;
    __asm__ volatile("cpuid" : "=a"(a), "=b"(b), "=c"(c), "=d"(d) : "a"(0), "c"(0));
    if (a < 7) return false;
    __asm__ volatile("cpuid" : "=a"(a), "=b"(b), "=c"(c), "=d"(d) : "a"(1), "c"(0));
    const bool sse41 = (c >> 19) & 1u, ssse3 = (c >> 9) & 1u;
    __asm__ volatile("cpuid" : "=a"(a), "=b"(b), "=c"(c), "=d"(d) : "a"(7), "c"(0));
    return sse41 && ssse3 && ((b >> 29) & 1u);
}

}  // namespace

Sha256::Sha256(int impl) {
    static const bool has_ni = cpu_has_shani();
    ni_ = impl == 1 ? false : impl == 2 ? has_ni : has_ni;
    const uint32_t init[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                              0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    memcpy(h_, init, sizeof h_);
}

void Sha256::compress(const uint8_t* p, size_t blocks) {
    if (ni_) blocks_shani(h_, p, blocks);
    else blocks_portable(h_, p, blocks);
}

void Sha256::update(const void* data, size_t n) {
    const uint8_t* p = static_cast<const uint8_t*>(data);
    total_ += n;
    if (fill_ > 0) {
        const size_t take = n < 64 - fill_ ? n : 64 - fill_;
        memcpy(buf_ + fill_, p, take);
        fill_ += take;
        p += take;
        n -= take;
        if (fill_ < 64) return;
        compress(buf_, 1);
        fill_ = 0;
    }
    if (n >= 64) {
        compress(p, n / 64);
        p += n / 64 * 64;
        n %= 64;
    }
    memcpy(buf_, p, n);
    fill_ = n;
}

void Sha256::final_hex(char out[65]) {
    const uint64_t bits = total_ * 8;
    const uint8_t one = 0x80, zero = 0;
    update(&one, 1);
    while (fill_ != 56) update(&zero, 1);
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = static_cast<uint8_t>(bits >> (56 - 8 * i));
    update(len, 8);
    static const char* digits = "0123456789abcdef";
    for (int i = 0; i < 8; ++i)
        for (int k = 0; k < 8; ++k) out[8 * i + k] = digits[(h_[i] >> (28 - 4 * k)) & 0xf];
    out[64] = '\0';
}

// ---- streaming tensor data ----

namespace {

constexpr size_t kStage = size_t{64} << 20;  // bytes per pinned buffer
constexpr size_t kAlign = 64;                // tensor alignment of both file formats

struct Piece {
    const void* src;  // nullptr: zero padding
    size_t bytes;
    bool device;
};

// The pieces of the data section: each tensor's bytes, then zeros to the next multiple of 64.
std::vector<Piece> pieces_of(const TensorSource* tensors, size_t n) {
    std::vector<Piece> out;
    for (size_t i = 0; i < n; ++i) {
        const size_t bytes = static_cast<size_t>(tensors[i].numel) * sizeof(float);
        if (bytes > 0) out.push_back(Piece{tensors[i].data, bytes, tensors[i].device});
        const size_t pad = (kAlign - bytes % kAlign) % kAlign;
        if (pad > 0) out.push_back(Piece{nullptr, pad, false});
    }
    return out;
}

struct PinnedPair {
    void* buf[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    ~PinnedPair() {
        for (int i = 0; i < 2; ++i) {
            if (done[i]) (void)hipEventDestroy(done[i]);
            if (buf[i]) (void)hipHostFree(buf[i]);
        }
    }
    int init() {
        for (int i = 0; i < 2; ++i) {
            DLLM_TRY(check_hip(hipHostMalloc(&buf[i], kStage, hipHostMallocDefault), "pinned staging buffer"));
            DLLM_TRY(check_hip(hipEventCreateWithFlags(&done[i], hipEventDisableTiming), "event"));
        }
        return kOk;
    }
};

}  // namespace

int stream_tensor_data(const TensorSource* tensors, size_t n, FILE* file, char hex[65], hipStream_t stream) {
    const std::vector<Piece> pieces = pieces_of(tensors, n);
    bool any_device = false;
    for (const Piece& p : pieces) any_device = any_device || p.device;
    Sha256 sha;
    if (!any_device) {  // host data: hash and write in place
        static const uint8_t zeros[kAlign] = {};
        for (const Piece& p : pieces) {
            const void* src = p.src ? p.src : zeros;
            sha.update(src, p.bytes);
            if (file && fwrite(src, 1, p.bytes, file) != p.bytes) return fail(kInvalidArgument, "file write failed");
        }
        sha.final_hex(hex);
        return kOk;
    }
    PinnedPair pin;
    DLLM_TRY(pin.init());
    // fill(k) packs the next kStage bytes of the pieces into buffer k: device pieces by async copies on `stream`,
    // host pieces and padding by the host
    size_t piece = 0, within = 0;
    auto fill = [&](int k, size_t* used) -> int {
        char* dst = static_cast<char*>(pin.buf[k]);
        size_t off = 0;
        while (piece < pieces.size() && off < kStage) {
            const Piece& p = pieces[piece];
            const size_t take = p.bytes - within < kStage - off ? p.bytes - within : kStage - off;
            if (!p.src) memset(dst + off, 0, take);
            else if (p.device)
                DLLM_TRY(check_hip(hipMemcpyAsync(dst + off, static_cast<const char*>(p.src) + within, take,
                                                  hipMemcpyDeviceToHost, stream),
                                   "device to host copy"));
            else memcpy(dst + off, static_cast<const char*>(p.src) + within, take);
            off += take;
            within += take;
            if (within == p.bytes) {
                ++piece;
                within = 0;
            }
        }
        *used = off;
        return check_hip(hipEventRecord(pin.done[k], stream), "event record");
    };
    size_t used[2] = {0, 0};
    DLLM_TRY(fill(0, &used[0]));
    for (int k = 0;; k ^= 1) {
        const bool more = piece < pieces.size();
        if (more) DLLM_TRY(fill(k ^ 1, &used[k ^ 1]));  // the next buffer's copies run while this one is hashed
        DLLM_TRY(check_hip(hipEventSynchronize(pin.done[k]), "event wait"));
        sha.update(pin.buf[k], used[k]);
        if (file && fwrite(pin.buf[k], 1, used[k], file) != used[k]) return fail(kInvalidArgument, "file write failed");
        if (!more) break;
    }
    sha.final_hex(hex);
    return kOk;
}

int write_tensor_file(const char* path, int kind, const char* header, size_t header_len, const TensorSource* tensors,
                      size_t n, char hex[65], hipStream_t stream) {
    DLLM_REQUIRE(path && header && hex, "null argument");
    DLLM_REQUIRE(kind == kModelFile || kind == kCheckpointFile, "kind must be 0 (model.dllm) or 1 (.dllmckpt)");
    const std::string placeholder = "\"fingerprint\":\"" + std::string(64, '0') + "\"";
    const std::string head(header, header_len);
    const size_t mark = head.find(placeholder);
    DLLM_REQUIRE(mark != std::string::npos, "the header has no \"fingerprint\" placeholder of 64 zeros");
    // prefix: magic, format version 1, header length (modelfile.py:30-33, trainer.py:86-90)
    const std::string magic = kind == kModelFile ? std::string("DLLM") : std::string("DLLMCKPT");
    const size_t prefix = magic.size() + 4 + 8;
    const size_t pad = (kAlign - (prefix + header_len) % kAlign) % kAlign;
    const uint64_t padded_len = header_len + pad;
    FILE* f = fopen(path, "wb+");
    DLLM_REQUIRE(f, std::string("cannot open ") + path);
    std::vector<uint8_t> pre(prefix);
    memcpy(pre.data(), magic.data(), magic.size());
    const uint32_t version = 1;
    for (int i = 0; i < 4; ++i) pre[magic.size() + i] = static_cast<uint8_t>(version >> (8 * i));
    for (int i = 0; i < 8; ++i) pre[magic.size() + 4 + i] = static_cast<uint8_t>(padded_len >> (8 * i));
    const std::string spaces(pad, ' ');
    int status = kOk;
    if (fwrite(pre.data(), 1, prefix, f) != prefix || fwrite(header, 1, header_len, f) != header_len ||
        fwrite(spaces.data(), 1, pad, f) != pad)
        status = fail(kInvalidArgument, "file write failed");
    if (status == kOk) status = stream_tensor_data(tensors, n, f, hex, stream);
    if (status == kOk) {  // patch the fingerprint into the header
        const long at = static_cast<long>(prefix + mark + strlen("\"fingerprint\":\""));
        if (fseek(f, at, SEEK_SET) != 0 || fwrite(hex, 1, 64, f) != 64)
            status = fail(kInvalidArgument, "file write failed");
    }
    if (fclose(f) != 0 && status == kOk) status = fail(kInvalidArgument, "file close failed");
    return status;
}

int read_tensor_file_data(const char* path, int kind, const TensorSource* tensors, size_t n, char hex[65],
                          int load, hipStream_t stream) {
    DLLM_REQUIRE(path && hex, "null argument");
    FILE* f = fopen(path, "rb");
    DLLM_REQUIRE(f, std::string("cannot open ") + path);
    const size_t magic_len = kind == kModelFile ? 4 : 8;
    uint8_t pre[20];
    int status = kOk;
    if (fread(pre, 1, magic_len + 12, f) != magic_len + 12) status = fail(kInvalidArgument, "not a tensor file");
    uint64_t header_len = 0;
    if (status == kOk) {
        for (int i = 0; i < 8; ++i) header_len |= uint64_t{pre[magic_len + 4 + i]} << (8 * i);
        if (fseek(f, static_cast<long>(magic_len + 12 + header_len), SEEK_SET) != 0)
            status = fail(kInvalidArgument, "truncated header");
    }
    // the data section: hashed whole; with `load`, each tensor's bytes go to its destination as they pass
    std::vector<Piece> pieces = pieces_of(tensors, n);
    bool any_device = false;
    for (const Piece& p : pieces) any_device = any_device || p.device;
    PinnedPair pin;  // pinned buffers only when bytes go to the device
    std::vector<char> plain;
    if (status == kOk && load && any_device) {
        status = pin.init();
    } else if (status == kOk) {
        plain.resize(2 * kStage);
        pin.buf[0] = plain.data();
        pin.buf[1] = plain.data() + kStage;
    }
    Sha256 sha;
    size_t piece = 0, within = 0;
    bool short_data = false;
    for (int k = 0; status == kOk; k ^= 1) {
        if (pin.done[k]) DLLM_TRY(check_hip(hipEventSynchronize(pin.done[k]), "event wait"));  // its uploads are done
        const size_t got = fread(pin.buf[k], 1, kStage, f);
        if (got == 0) break;
        sha.update(pin.buf[k], got);
        if (load) {
            size_t off = 0;
            while (off < got && piece < pieces.size()) {
                const Piece& p = pieces[piece];
                const size_t take = p.bytes - within < got - off ? p.bytes - within : got - off;
                if (p.src && p.device)
                    status = check_hip(hipMemcpyAsync(const_cast<char*>(static_cast<const char*>(p.src)) + within,
                                                      static_cast<char*>(pin.buf[k]) + off, take,
                                                      hipMemcpyHostToDevice, stream),
                                       "host to device copy");
                else if (p.src)
                    memcpy(const_cast<char*>(static_cast<const char*>(p.src)) + within,
                           static_cast<char*>(pin.buf[k]) + off, take);
                off += take;
                within += take;
                if (within == p.bytes) {
                    ++piece;
                    within = 0;
                }
            }
            if (status == kOk && pin.done[k]) status = check_hip(hipEventRecord(pin.done[k], stream), "event record");
        }
    }
    if (load && status == kOk && piece < pieces.size()) short_data = true;
    fclose(f);
    if (!pin.done[0]) pin.buf[0] = pin.buf[1] = nullptr;  // plain host buffers: not freed by PinnedPair
    DLLM_TRY(status);
    if (load && any_device) DLLM_TRY(check_hip(hipStreamSynchronize(stream), "stream sync"));
    DLLM_REQUIRE(!short_data, "the file holds fewer tensor bytes than the tensors need");
    sha.final_hex(hex);
    return kOk;
}

}  // namespace dllm_hip

extern "C" {

int dllm_hip_sha256(const void* data, size_t n, int impl, char* hex_out) {
    DLLM_REQUIRE((data || n == 0) && hex_out, "null argument");
    DLLM_REQUIRE(impl >= 0 && impl <= 2, "impl must be 0 (best), 1 (portable) or 2 (SHA extensions if present)");
    dllm_hip::Sha256 sha(impl);
    sha.update(data, n);
    sha.final_hex(hex_out);
    return dllm_hip::kOk;
}

int dllm_hip_write_tensor_file(const char* path, int kind, const char* header, size_t header_len,
                               const float* const* host_tensors, const int64_t* numels, size_t count, char* hex_out) {
    DLLM_REQUIRE(count == 0 || (host_tensors && numels), "null argument");
    std::vector<dllm_hip::TensorSource> t(count);
    for (size_t i = 0; i < count; ++i) t[i] = dllm_hip::TensorSource{host_tensors[i], numels[i], false};
    return dllm_hip::write_tensor_file(path, kind, header, header_len, t.data(), count, hex_out, nullptr);
}

int dllm_hip_tensor_file_fingerprint(const char* path, int kind, char* hex_out) {
    return dllm_hip::read_tensor_file_data(path, kind, nullptr, 0, hex_out, 0, nullptr);
}

}  // extern "C"
