// Kernel metadata read from an AMDGPU code object on the host.
//
// The reference's loader takes the kernel's workgroup size and LDS from the
// caller (KernelLoadConfig, src/kfd/mod.rs:2559-2651) and knows each kernel's
// argument size from the kernel it generated (T0Kernel::kernarg_size,
// src/t0/compile.rs:495-510).  A code object handed to t0g_kernel_load comes
// from anywhere, so its argument size is read from the code object itself:
// the NT_AMDGPU_METADATA note of the gfx950 ELF (a MessagePack map whose
// "amdhsa.kernels" array lists every kernel's ".args", ".kernarg_segment_size",
// ".group_segment_fixed_size" and ".max_flat_workgroup_size").  The input may
// be a bare ELF or a clang offload bundle (hipcc --genco output).  Every read
// is bounds-checked: the bytes are untrusted.
#include <stdint.h>
#include <string.h>

#include <string>

#include "t0g_internal.h"

namespace t0g {

namespace {

uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t le32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
uint64_t le64(const uint8_t *p) { return (uint64_t)le32(p) | ((uint64_t)le32(p + 4) << 32); }

constexpr uint16_t kEmAmdgpu = 224;
constexpr uint32_t kMachMask = 0xff;
constexpr uint32_t kMachGfx950 = 0x4f;
constexpr uint32_t kShtNote = 7;
constexpr uint32_t kNtAmdgpuMetadata = 32;
constexpr char kBundleMagic[] = "__CLANG_OFFLOAD_BUNDLE__";

// The gfx950 ELF inside a code object: the object itself, or the bundle entry
// whose target id names gfx950.
int find_elf(const uint8_t *p, size_t n, const uint8_t **elf, size_t *elf_n) {
    if (n >= 4 && memcmp(p, "\x7f" "ELF", 4) == 0) {
        *elf = p;
        *elf_n = n;
        return T0G_OK;
    }
    const size_t magic = sizeof kBundleMagic - 1;
    if (n < magic + 8 || memcmp(p, kBundleMagic, magic) != 0)
        return fail(T0G_ERR_INVALID_ARG, "code object is neither an ELF nor a clang offload bundle");
    const uint64_t entries = le64(p + magic);
    size_t pos = magic + 8;
    for (uint64_t i = 0; i < entries; ++i) {
        if (n - pos < 24) break;
        const uint64_t off = le64(p + pos), size = le64(p + pos + 8), id_len = le64(p + pos + 16);
        pos += 24;
        if (id_len > n - pos) break;
        const std::string id((const char *)p + pos, (size_t)id_len);
        pos += (size_t)id_len;
        if (id.find("amdgcn") == std::string::npos || id.find("gfx950") == std::string::npos) continue;
        if (off > n || size > n - off || size < 4)
            return fail(T0G_ERR_INVALID_ARG, "offload bundle entry '%s' lies outside the %zu-byte object", id.c_str(), n);
        if (memcmp(p + off, "\x7f" "ELF", 4) != 0)
            return fail(T0G_ERR_INVALID_ARG, "offload bundle entry '%s' is not an ELF (compressed bundles are not read)",
                        id.c_str());
        *elf = p + off;
        *elf_n = (size_t)size;
        return T0G_OK;
    }
    return fail(T0G_ERR_INVALID_ARG, "offload bundle has no gfx950 code object");
}

// MessagePack reader: every accessor returns false past the end or on a type
// it does not take.
class Msgpack {
  public:
    Msgpack(const uint8_t *p, size_t n) : p_(p), end_(p + n) {}

    bool map(uint32_t *count) {
        uint8_t t;
        if (!byte(&t)) return false;
        if ((t & 0xf0) == 0x80) return (*count = t & 0x0f), true;
        if (t == 0xde) return be(2, count);
        if (t == 0xdf) return be(4, count);
        return false;
    }
    bool array(uint32_t *count) {
        uint8_t t;
        if (!byte(&t)) return false;
        if ((t & 0xf0) == 0x90) return (*count = t & 0x0f), true;
        if (t == 0xdc) return be(2, count);
        if (t == 0xdd) return be(4, count);
        return false;
    }
    bool str(std::string *s) {
        uint8_t t;
        uint32_t len;
        if (!byte(&t)) return false;
        if ((t & 0xe0) == 0xa0) len = t & 0x1f;
        else if (t == 0xd9 || t == 0xc4) { if (!be(1, &len)) return false; }
        else if (t == 0xda || t == 0xc5) { if (!be(2, &len)) return false; }
        else if (t == 0xdb || t == 0xc6) { if (!be(4, &len)) return false; }
        else return false;
        if ((size_t)(end_ - p_) < len) return false;
        s->assign((const char *)p_, len);
        p_ += len;
        return true;
    }
    bool uint(uint64_t *v) {
        uint8_t t;
        if (!byte(&t)) return false;
        if (t <= 0x7f) return (*v = t), true;
        int bytes = 0;
        bool is_signed = false;
        switch (t) {
            case 0xcc: bytes = 1; break;
            case 0xcd: bytes = 2; break;
            case 0xce: bytes = 4; break;
            case 0xcf: bytes = 8; break;
            case 0xd0: bytes = 1; is_signed = true; break;
            case 0xd1: bytes = 2; is_signed = true; break;
            case 0xd2: bytes = 4; is_signed = true; break;
            case 0xd3: bytes = 8; is_signed = true; break;
            default: return false;
        }
        if ((size_t)(end_ - p_) < (size_t)bytes) return false;
        uint64_t x = 0;
        for (int i = 0; i < bytes; ++i) x = (x << 8) | p_[i];
        p_ += bytes;
        if (is_signed && (x >> (8 * bytes - 1)) & 1) return false;   // negative
        *v = x;
        return true;
    }
    bool skip(int depth = 0) {
        if (depth > 32 || p_ >= end_) return false;
        const uint8_t t = *p_;
        uint32_t count;
        if ((t & 0xf0) == 0x80 || t == 0xde || t == 0xdf) {
            if (!map(&count)) return false;
            for (uint64_t i = 0; i < 2ull * count; ++i)
                if (!skip(depth + 1)) return false;
            return true;
        }
        if ((t & 0xf0) == 0x90 || t == 0xdc || t == 0xdd) {
            if (!array(&count)) return false;
            for (uint32_t i = 0; i < count; ++i)
                if (!skip(depth + 1)) return false;
            return true;
        }
        std::string s;
        uint64_t u;
        if ((t & 0xe0) == 0xa0 || (t >= 0xd9 && t <= 0xdb) || (t >= 0xc4 && t <= 0xc6)) return str(&s);
        if (t <= 0x7f || (t >= 0xcc && t <= 0xcf)) return uint(&u);
        size_t len;
        if (t >= 0xe0 || t == 0xc0 || t == 0xc2 || t == 0xc3) len = 1;             // negative fixint, nil, bool
        else if (t >= 0xd0 && t <= 0xd3) len = 1 + (1u << (t - 0xd0));           // int8..int64
        else if (t == 0xca) len = 5;                                                // float32
        else if (t == 0xcb) len = 9;                                                // float64
        else return false;                                                          // ext types: not in this metadata
        if ((size_t)(end_ - p_) < len) return false;
        p_ += len;
        return true;
    }

  private:
    bool byte(uint8_t *t) {
        if (p_ >= end_) return false;
        *t = *p_++;
        return true;
    }
    bool be(int bytes, uint32_t *v) {
        if ((size_t)(end_ - p_) < (size_t)bytes) return false;
        uint32_t x = 0;
        for (int i = 0; i < bytes; ++i) x = (x << 8) | p_[i];
        p_ += bytes;
        *v = x;
        return true;
    }
    const uint8_t *p_, *end_;
};

bool fits_u32(uint64_t v, uint32_t *out) {
    if (v > 0xffffffffull) return false;
    *out = (uint32_t)v;
    return true;
}

// One entry of "amdhsa.kernels".  *matched: its ".name" is `symbol`.
bool read_kernel(Msgpack &mp, const char *symbol, bool *matched, KernelMeta *meta) {
    uint32_t keys;
    if (!mp.map(&keys)) return false;
    KernelMeta km;
    memset(&km, 0, sizeof km);
    bool named = false;
    for (uint32_t i = 0; i < keys; ++i) {
        std::string key;
        if (!mp.str(&key)) return false;
        uint64_t v = 0;
        if (key == ".name") {
            std::string name;
            if (!mp.str(&name)) return false;
            named = name == symbol;
        } else if (key == ".kernarg_segment_size") {
            if (!mp.uint(&v) || !fits_u32(v, &km.kernarg_segment_size)) return false;
        } else if (key == ".group_segment_fixed_size") {
            if (!mp.uint(&v) || !fits_u32(v, &km.group_segment_size)) return false;
        } else if (key == ".private_segment_fixed_size") {
            if (!mp.uint(&v) || !fits_u32(v, &km.private_segment_size)) return false;
        } else if (key == ".max_flat_workgroup_size") {
            if (!mp.uint(&v) || !fits_u32(v, &km.max_workgroup_size)) return false;
        } else if (key == ".wavefront_size") {
            if (!mp.uint(&v) || !fits_u32(v, &km.wavefront_size)) return false;
        } else if (key == ".args") {
            uint32_t n_args;
            if (!mp.array(&n_args)) return false;
            for (uint32_t a = 0; a < n_args; ++a) {
                uint32_t fields;
                if (!mp.map(&fields)) return false;
                uint64_t off = 0, size = 0;
                std::string kind;
                for (uint32_t f = 0; f < fields; ++f) {
                    std::string fk;
                    if (!mp.str(&fk)) return false;
                    if (fk == ".offset") { if (!mp.uint(&off)) return false; }
                    else if (fk == ".size") { if (!mp.uint(&size)) return false; }
                    else if (fk == ".value_kind") { if (!mp.str(&kind)) return false; }
                    else if (!mp.skip()) return false;
                }
                // hidden_* arguments are filled in by the HIP runtime after the caller's block
                if (kind.compare(0, 7, "hidden_") != 0 && off + size > km.explicit_args_size) {
                    if (off + size > 0xffffffffull) return false;
                    km.explicit_args_size = (uint32_t)(off + size);
                }
            }
        } else if (!mp.skip()) {
            return false;
        }
    }
    *matched = named;
    if (named) *meta = km;
    return true;
}

}  // namespace

int read_kernel_meta(const void *code_object, size_t size, const char *symbol, KernelMeta *out) {
    if (!code_object || !symbol || !out) return fail(T0G_ERR_INVALID_ARG, "NULL argument");
    const uint8_t *elf = nullptr;
    size_t n = 0;
    int rc = find_elf((const uint8_t *)code_object, size, &elf, &n);
    if (rc) return rc;
    if (n < 64 || elf[4] != 2 || elf[5] != 1)
        return fail(T0G_ERR_INVALID_ARG, "code object is not a little-endian 64-bit ELF");
    if (le16(elf + 18) != kEmAmdgpu) return fail(T0G_ERR_INVALID_ARG, "ELF machine %u is not AMDGPU", le16(elf + 18));
    const uint32_t mach = le32(elf + 0x30) & kMachMask;
    if (mach != kMachGfx950)
        return fail(T0G_ERR_UNSUPPORTED_CONFIG, "code object is built for AMDGPU mach 0x%02x, not gfx950 (0x4f)", mach);
    const uint64_t shoff = le64(elf + 0x28);
    const uint16_t shentsize = le16(elf + 0x3a), shnum = le16(elf + 0x3c);
    if (shentsize < 64 || shoff > n || (uint64_t)shnum * shentsize > n - shoff)
        return fail(T0G_ERR_INVALID_ARG, "ELF section table lies outside the object");
    bool saw_metadata = false;
    for (uint16_t s = 0; s < shnum; ++s) {
        const uint8_t *sh = elf + shoff + (uint64_t)s * shentsize;
        if (le32(sh + 4) != kShtNote) continue;
        const uint64_t off = le64(sh + 0x18), sz = le64(sh + 0x20);
        if (off > n || sz > n - off) return fail(T0G_ERR_INVALID_ARG, "ELF note section lies outside the object");
        uint64_t pos = 0;
        while (sz - pos >= 12) {
            const uint8_t *note = elf + off + pos;
            const uint32_t namesz = le32(note), descsz = le32(note + 4), type = le32(note + 8);
            const uint64_t name_pad = ((uint64_t)namesz + 3) & ~3ull, desc_pad = ((uint64_t)descsz + 3) & ~3ull;
            if (name_pad + desc_pad > sz - pos - 12) return fail(T0G_ERR_INVALID_ARG, "truncated ELF note");
            const char *name = (const char *)note + 12;
            const uint8_t *desc = note + 12 + name_pad;
            pos += 12 + name_pad + desc_pad;
            if (type != kNtAmdgpuMetadata || namesz != 7 || memcmp(name, "AMDGPU", 7) != 0) continue;
            saw_metadata = true;
            Msgpack mp(desc, descsz);
            uint32_t top;
            if (!mp.map(&top)) return fail(T0G_ERR_INVALID_ARG, "malformed AMDGPU metadata");
            for (uint32_t i = 0; i < top; ++i) {
                std::string key;
                if (!mp.str(&key)) return fail(T0G_ERR_INVALID_ARG, "malformed AMDGPU metadata");
                if (key != "amdhsa.kernels") {
                    if (!mp.skip()) return fail(T0G_ERR_INVALID_ARG, "malformed AMDGPU metadata");
                    continue;
                }
                uint32_t kernels;
                if (!mp.array(&kernels)) return fail(T0G_ERR_INVALID_ARG, "malformed amdhsa.kernels");
                for (uint32_t k = 0; k < kernels; ++k) {
                    bool matched = false;
                    KernelMeta km;
                    if (!read_kernel(mp, symbol, &matched, &km))
                        return fail(T0G_ERR_INVALID_ARG, "malformed entry %u of amdhsa.kernels", k);
                    if (matched) {
                        *out = km;
                        return T0G_OK;
                    }
                }
            }
        }
    }
    if (!saw_metadata) return fail(T0G_ERR_INVALID_ARG, "code object has no AMDGPU metadata note");
    return fail(T0G_ERR_INVALID_ARG, "code object has no kernel named '%s'", symbol);
}

}  // namespace t0g

extern "C" int t0g_code_object_kernel_meta(const void *code_object, size_t size, const char *symbol,
                                           t0g_kernel_meta *out) {
    if (!out) return t0g::fail(T0G_ERR_INVALID_ARG, "NULL argument");
    t0g::KernelMeta km;
    int rc = t0g::read_kernel_meta(code_object, size, symbol, &km);
    if (rc) return rc;
    out->kernarg_size = km.explicit_args_size;
    out->kernarg_segment_size = km.kernarg_segment_size;
    out->group_segment_size = km.group_segment_size;
    out->private_segment_size = km.private_segment_size;
    out->max_workgroup_size = km.max_workgroup_size;
    out->wavefront_size = km.wavefront_size;
    return t0g::ok();
}
