// .sfe GPU packages of a compiled decoder plan: save, inspect, load.
//
// Modelled on the reference's AOT package format 1 (src/aot_runtime.cpp:217-316;
// docs/AOT_DEPLOYMENT.md:6-35): a directory with a .sfe suffix written through a
// temporary directory and renamed into place, a key=value manifest ('#'
// comments, duplicate keys rejected; parse_fields, aot_runtime.cpp:97-121), FNV-1a
// 64-bit checksums of every file (26-35), and a loader that validates the
// manifest, the files and the library's embedded metadata before any call
// (167-199, 301-316) and rejects a mismatch rather than recompiling.
//
// What a GPU plan adds over the reference's single CPU kernel: the gfx950 code
// objects (the device half of libsfg_hip.so, extracted from its offload bundles
// so they can be inspected and checksummed on their own), and the plan's
// packed device constants (the reference lists packed-constant relocation as
// future work, docs/AOT_DEPLOYMENT.md:44-49).
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <map>
#include <sstream>
#include <type_traits>

#include "sfg_decoder.hpp"
#include "sfg_runtime_internal.hpp"

namespace schedforge::hip {
namespace {

constexpr const char* kVersion = "0.9.0";
constexpr const char* kAbi = "sfg_hip_decoder_layer_v1";
constexpr const char* kTarget = "gfx950";
constexpr std::size_t kAlign = 256;

// FNV-1a, 64-bit: offset basis 0xcbf29ce484222325, prime 0x100000001b3.
struct Fnv1a64 {
    std::uint64_t h = 0xcbf29ce484222325ULL;
    void update(const void* data, std::size_t bytes) {
        const auto* p = static_cast<const unsigned char*>(data);
        for (std::size_t i = 0; i < bytes; ++i) {
            h ^= p[i];
            h *= 0x100000001b3ULL;
        }
    }
    std::string hex() const {
        char buf[17];
        std::snprintf(buf, sizeof buf, "%016llx", static_cast<unsigned long long>(h));
        return buf;
    }
};

std::string read_file(const std::filesystem::path& path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) throw std::runtime_error("cannot read .sfe package file: " + path.string());
    return {std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>()};
}

void write_file(const std::filesystem::path& path, const void* data, std::size_t bytes) {
    std::ofstream out(path, std::ios::binary | std::ios::trunc);
    if (!out) throw std::runtime_error("cannot write .sfe package file: " + path.string());
    out.write(static_cast<const char*>(data), static_cast<std::streamsize>(bytes));
    if (!out) throw std::runtime_error("failed writing .sfe package file: " + path.string());
}

DecoderPackageFile describe_file(const std::filesystem::path& root, const std::string& rel) {
    const std::string content = read_file(root / rel);
    return {rel, content.size(), package_checksum(content.data(), content.size())};
}

// ------------------------------------------------------------ manifest fields

std::map<std::string, std::string> parse_fields(const std::string& text) {
    std::map<std::string, std::string> fields;
    std::istringstream in(text);
    std::string line;
    while (std::getline(in, line)) {
        if (line.empty() || line.front() == '#') continue;
        const auto eq = line.find('=');
        if (eq == std::string::npos || eq == 0)
            throw std::runtime_error("invalid .sfe manifest line: " + line);
        if (!fields.emplace(line.substr(0, eq), line.substr(eq + 1)).second)
            throw std::runtime_error("duplicate .sfe manifest field: " + line.substr(0, eq));
    }
    return fields;
}

const std::string& required(const std::map<std::string, std::string>& f, const std::string& key) {
    const auto it = f.find(key);
    if (it == f.end()) throw std::runtime_error("missing .sfe manifest field: " + key);
    return it->second;
}

template <typename T>
T number(const std::map<std::string, std::string>& f, const std::string& key) {
    const std::string& s = required(f, key);
    try {
        std::size_t used = 0;
        T v;
        if constexpr (std::is_same_v<T, float>) v = std::stof(s, &used);
        else if constexpr (std::is_same_v<T, std::size_t>) v = static_cast<T>(std::stoull(s, &used));
        else v = static_cast<T>(std::stoll(s, &used));
        if (used != s.size()) throw std::invalid_argument(s);
        return v;
    } catch (const std::exception&) {
        throw std::runtime_error("malformed .sfe manifest field: " + key + "=" + s);
    }
}

std::vector<std::string> split(const std::string& s, char sep) {
    std::vector<std::string> parts;
    std::string item;
    std::istringstream in(s);
    while (std::getline(in, item, sep)) parts.push_back(item);
    if (!s.empty() && s.back() == sep) parts.emplace_back();
    return parts;
}

std::string float_text(float v) {
    char buf[32];
    std::snprintf(buf, sizeof buf, "%.9g", static_cast<double>(v));  // round-trips a float
    return buf;
}

// "path,bytes,checksum"
std::string file_text(const DecoderPackageFile& f) {
    return f.path + "," + std::to_string(f.bytes) + "," + f.checksum;
}

DecoderPackageFile parse_file(const std::string& key, const std::string& value) {
    const auto parts = split(value, ',');
    if (parts.size() != 3 || parts[0].empty() || parts[2].size() != 16)
        throw std::runtime_error("malformed .sfe manifest field: " + key + "=" + value);
    DecoderPackageFile f;
    f.path = parts[0];
    f.checksum = parts[2];
    try {
        f.bytes = std::stoull(parts[1]);
    } catch (const std::exception&) {
        throw std::runtime_error("malformed .sfe manifest field: " + key + "=" + value);
    }
    // Package-relative paths only.
    const std::filesystem::path p(f.path);
    if (p.is_absolute() || std::any_of(p.begin(), p.end(), [](const auto& c) { return c == ".."; }))
        throw std::runtime_error("invalid .sfe package path: " + f.path);
    return f;
}

std::string shape_text(const std::vector<int>& s) {
    std::string out;
    for (std::size_t i = 0; i < s.size(); ++i) out += (i ? "x" : "") + std::to_string(s[i]);
    return out;
}

std::vector<int> parse_shape(const std::string& s) {
    std::vector<int> out;
    for (const auto& part : split(s, 'x')) out.push_back(std::stoi(part));
    return out;
}

// constant.<i>=name;logical;packed;layout;bytes
DecoderConstant parse_constant(const std::string& key, const std::string& value) {
    const auto parts = split(value, ';');
    try {
        if (parts.size() != 5) throw std::invalid_argument(value);
        DecoderConstant c;
        c.name = parts[0];
        c.logical_shape = parse_shape(parts[1]);
        c.packed_shape = parse_shape(parts[2]);
        c.layout = parts[3];
        c.bytes = std::stoull(parts[4]);
        return c;
    } catch (const std::exception&) {
        throw std::runtime_error("malformed .sfe manifest field: " + key + "=" + value);
    }
}

DecoderPrecision parse_precision(const std::string& s) {
    if (s == "f32") return DecoderPrecision::F32;
    if (s == "bf16") return DecoderPrecision::BF16;
    if (s == "w8") return DecoderPrecision::W8;
    throw std::runtime_error("unknown .sfe precision: " + s);
}

// ------------------------------------------------------------ plan buffers

// The weight-table slot of each named plan buffer (the names compile gives them).
void bind_buffer(sfg_layer_weights& w, const std::string& name, void* p) {
    auto* f = static_cast<const float*>(p);
    if (name == "rms1_weight") w.rms1 = f;
    else if (name == "rms2_weight") w.rms2 = f;
    else if (name == "packed_qkv_weight") w.w_qkv = p;
    else if (name == "packed_qkv_weight.scales") w.s_qkv = f;
    else if (name == "output_weight") w.w_o = p;
    else if (name == "output_weight.scales") w.s_o = f;
    else if (name == "packed_gate_up_weight") w.w_gate_up = p;
    else if (name == "packed_gate_up_weight.scales") w.s_gate_up = f;
    else if (name == "down_weight") w.w_down = p;
    else if (name == "down_weight.scales") w.s_down = f;
    else if (name == "router_weight") w.router = f;
    else if (name == "router_bias") w.router_bias = f;
    else if (name == "expert_w13") w.w13 = p;
    else if (name == "expert_w13.scales") w.s13 = f;
    else if (name == "expert_w2") w.w2 = p;
    else if (name == "expert_w2.scales") w.s2 = f;
    else if (name == "k_pool") w.k_pool = p;
    else if (name == "v_pool") w.v_pool = p;
    else if (name == "page_table") w.page_table = static_cast<const std::int32_t*>(p);
    else if (name == "rope_table") w.rope_table = f;
    else throw std::runtime_error("unknown .sfe plan buffer: " + name);
}

constexpr const char* kTraceIds = "routing_trace.ids";
constexpr const char* kTraceWeights = "routing_trace.weights";

std::uint16_t read_u16(const std::string& s, std::size_t at) {
    std::uint16_t v;
    std::memcpy(&v, s.data() + at, 2);
    return v;
}
std::uint32_t read_u32(const std::string& s, std::size_t at) {
    std::uint32_t v;
    std::memcpy(&v, s.data() + at, 4);
    return v;
}
std::uint64_t read_u64(const std::string& s, std::size_t at) {
    std::uint64_t v;
    std::memcpy(&v, s.data() + at, 8);
    return v;
}

void require_range(const std::string& s, std::uint64_t at, std::uint64_t bytes, const char* what) {
    if (at > s.size() || bytes > s.size() - at)
        throw std::runtime_error(std::string("truncated library: ") + what);
}

// constants.bin in one streaming pass: the whole-file checksum and each
// buffer's own.
void check_constants(const std::filesystem::path& root, const DecoderPackageManifest& m) {
    std::ifstream in(root / m.constants.path, std::ios::binary);
    if (!in) throw std::runtime_error("cannot read .sfe package file: " + m.constants.path);
    std::vector<char> chunk(std::size_t{1} << 24);
    Fnv1a64 whole, part;
    std::size_t pos = 0, next = 0;
    std::string bad;  // first buffer whose checksum differs
    while (in) {
        in.read(chunk.data(), static_cast<std::streamsize>(chunk.size()));
        const std::size_t n = static_cast<std::size_t>(in.gcount());
        if (n == 0) break;
        whole.update(chunk.data(), n);
        std::size_t k = 0;
        while (k < n && next < m.buffers.size()) {
            const auto& b = m.buffers[next];
            const std::size_t at = pos + k;
            if (at + (n - k) <= b.offset) break;
            if (at < b.offset) k += b.offset - at;
            const std::size_t take = std::min(n - k, b.offset + b.bytes - (pos + k));
            part.update(chunk.data() + k, take);
            k += take;
            if (pos + k == b.offset + b.bytes) {
                if (part.hex() != b.checksum && bad.empty()) bad = b.name;
                part = Fnv1a64{};
                ++next;
            }
        }
        pos += n;
    }
    if (pos != m.constants.bytes || whole.hex() != m.constants.checksum)
        throw std::runtime_error(".sfe checksum mismatch: " + m.constants.path);
    if (next != m.buffers.size()) throw std::runtime_error(".sfe buffer table exceeds constants.bin");
    if (!bad.empty()) throw std::runtime_error(".sfe checksum mismatch: buffer " + bad);
}

// The package's code objects, checked against the ones embedded in `library`.
void check_code_objects(const std::filesystem::path& root, const DecoderPackageManifest& m) {
    const auto embedded = embedded_code_objects(root / m.library.path);
    if (embedded.size() != m.code_objects.size())
        throw std::runtime_error(".sfe code objects do not match the packaged library");
    for (std::size_t i = 0; i < embedded.size(); ++i) {
        const auto& e = embedded[i];
        const auto& c = m.code_objects[i];
        if (e.target_id != c.target_id || e.bytes.size() != c.file.bytes ||
            package_checksum(e.bytes.data(), e.bytes.size()) != c.file.checksum)
            throw std::runtime_error(".sfe code object " + c.file.path +
                                     " differs from the one embedded in the packaged library");
    }
}

}  // namespace

std::string package_checksum(const void* data, std::size_t bytes) {
    Fnv1a64 f;
    f.update(data, bytes);
    return f.hex();
}

// ------------------------------------------------------------ code objects

std::vector<EmbeddedCodeObject> embedded_code_objects(const std::filesystem::path& library) {
    const std::string elf = read_file(library);
    if (elf.size() < 64 || elf.compare(0, 4, "\x7f" "ELF") != 0 || elf[4] != 2 || elf[5] != 1)
        throw std::runtime_error("not a 64-bit little-endian ELF library: " + library.string());
    const std::uint64_t shoff = read_u64(elf, 0x28);
    const std::uint16_t shentsize = read_u16(elf, 0x3A), shnum = read_u16(elf, 0x3C),
                        shstrndx = read_u16(elf, 0x3E);
    if (shentsize < 64 || shstrndx >= shnum) throw std::runtime_error("malformed ELF section table");
    require_range(elf, shoff, static_cast<std::uint64_t>(shentsize) * shnum, "section table");
    auto section = [&](int i) { return shoff + static_cast<std::uint64_t>(i) * shentsize; };
    const std::uint64_t strtab = read_u64(elf, section(shstrndx) + 24);
    std::uint64_t fat_off = 0, fat_size = 0;
    bool found = false;
    for (int i = 0; i < shnum; ++i) {
        const std::uint64_t name = strtab + read_u32(elf, section(i));
        require_range(elf, name, 1, "section names");
        if (std::strncmp(elf.c_str() + name, ".hip_fatbin", 12) == 0) {
            fat_off = read_u64(elf, section(i) + 24);
            fat_size = read_u64(elf, section(i) + 32);
            found = true;
            break;
        }
    }
    if (!found) throw std::runtime_error("library has no .hip_fatbin section: " + library.string());
    require_range(elf, fat_off, fat_size, ".hip_fatbin");

    // Clang offload bundles: "__CLANG_OFFLOAD_BUNDLE__", u64 entry count, then
    // per entry u64 offset (from the bundle start), u64 size, u64 id length, id.
    static constexpr char kMagic[] = "__CLANG_OFFLOAD_BUNDLE__";
    constexpr std::size_t kMagicLen = sizeof kMagic - 1;
    std::vector<EmbeddedCodeObject> out;
    std::uint64_t pos = 0;
    while (pos + kMagicLen + 8 <= fat_size) {
        const std::uint64_t at = fat_off + pos;
        if (elf.compare(at, kMagicLen, kMagic) != 0) {
            pos += 8;
            continue;
        }
        const std::uint64_t entries = read_u64(elf, at + kMagicLen);
        std::uint64_t cursor = at + kMagicLen + 8, end = cursor;
        for (std::uint64_t e = 0; e < entries; ++e) {
            require_range(elf, cursor, 24, "offload bundle entry");
            const std::uint64_t off = read_u64(elf, cursor), size = read_u64(elf, cursor + 8),
                                id_len = read_u64(elf, cursor + 16);
            require_range(elf, cursor + 24, id_len, "offload bundle id");
            const std::string id = elf.substr(cursor + 24, id_len);
            cursor += 24 + id_len;
            require_range(elf, at + off, size, "offload bundle payload");
            if (size > 0 && id.find("amdgcn") != std::string::npos) {
                if (elf.compare(at + off, 4, "\x7f" "ELF") != 0)
                    throw std::runtime_error("code object " + id + " is not an uncompressed ELF");
                EmbeddedCodeObject co;
                co.target_id = id;
                co.bytes.assign(elf.begin() + static_cast<std::ptrdiff_t>(at + off),
                                elf.begin() + static_cast<std::ptrdiff_t>(at + off + size));
                out.push_back(std::move(co));
            }
            end = std::max(end, at + off + size);
        }
        pos = (std::max(end, cursor) - fat_off + 7) / 8 * 8;
    }
    if (out.empty()) throw std::runtime_error("library embeds no amdgcn code object: " + library.string());
    return out;
}

// ------------------------------------------------------------ manifest

std::string DecoderPackageManifest::dump() const {
    const DecoderConfig& c = config;
    std::ostringstream o;
    o << "# SchedForge GPU Executable\n"
      << "format_version=" << format_version << '\n'
      << "schedforge_version=" << schedforge_version << '\n'
      << "abi=" << abi << '\n'
      << "symbol=" << symbol << '\n'
      << "target=" << target << '\n'
      << "library_abi=" << library_abi << '\n'
      << "library_metadata=" << library_metadata << '\n'
      << "batch=" << c.batch << '\n'
      << "sequence=" << c.sequence << '\n'
      << "hidden=" << c.hidden << '\n'
      << "intermediate=" << c.intermediate << '\n'
      << "query_heads=" << c.query_heads << '\n'
      << "kv_heads=" << c.kv_heads << '\n'
      << "head_dim=" << c.head_dim << '\n'
      << "rms_epsilon=" << float_text(c.rms_epsilon) << '\n'
      << "rope_theta=" << float_text(c.rope_theta) << '\n'
      << "causal=" << (c.causal ? 1 : 0) << '\n'
      << "ffn=" << decoder_ffn_name(c.ffn) << '\n'
      << "experts=" << c.experts << '\n'
      << "top_k=" << c.top_k << '\n'
      << "context_sequence=" << c.context_sequence << '\n'
      << "precision=" << decoder_precision_name(c.precision) << '\n'
      << "page_tokens=" << c.page_tokens << '\n'
      << "weight_layout=" << policy.weight_layout << '\n'
      << "kv_splits=" << policy.kv_splits << '\n'
      << "gemm_tile=" << policy.gemm_tile << '\n'
      << "attn_waves=" << policy.attn_waves << '\n'
      << "pages_per_seq=" << pages_per_seq << '\n'
      << "num_pages=" << num_pages << '\n'
      << "routing_trace=" << (routing_trace ? 1 : 0) << '\n'
      << "workspace_bytes=" << workspace_bytes << '\n'
      << "naive_bytes=" << naive_bytes << '\n'
      << "plan=" << file_text(plan) << '\n'
      << "library=" << file_text(library) << '\n'
      << "constants=" << file_text(constants) << '\n'
      << "code_objects=" << code_objects.size() << '\n';
    for (std::size_t i = 0; i < code_objects.size(); ++i)
        o << "code_object." << i << '=' << file_text(code_objects[i].file) << ','
          << code_objects[i].target_id << '\n';
    o << "buffers=" << buffers.size() << '\n';
    for (std::size_t i = 0; i < buffers.size(); ++i)
        o << "buffer." << i << '=' << buffers[i].name << ',' << buffers[i].offset << ','
          << buffers[i].bytes << ',' << buffers[i].checksum << '\n';
    o << "constant_table=" << constant_table.size() << '\n';
    for (std::size_t i = 0; i < constant_table.size(); ++i) {
        const auto& k = constant_table[i];
        o << "constant." << i << '=' << k.name << ';' << shape_text(k.logical_shape) << ';'
          << shape_text(k.packed_shape) << ';' << k.layout << ';' << k.bytes << '\n';
    }
    return o.str();
}

DecoderPackageManifest DecoderPackageManifest::parse(const std::string& text) {
    const auto f = parse_fields(text);
    DecoderPackageManifest m;
    m.format_version = number<int>(f, "format_version");
    if (m.format_version != 1)
        throw std::runtime_error("unsupported .sfe format version: " + std::to_string(m.format_version));
    m.schedforge_version = required(f, "schedforge_version");
    m.abi = required(f, "abi");
    m.symbol = required(f, "symbol");
    if (m.abi != kAbi || m.symbol != m.abi) throw std::runtime_error("unsupported .sfe ABI: " + m.abi);
    m.target = required(f, "target");
    if (m.target != kTarget) throw std::runtime_error("unsupported .sfe target: " + m.target);
    m.library_abi = number<int>(f, "library_abi");
    m.library_metadata = required(f, "library_metadata");
    DecoderConfig& c = m.config;
    c.batch = number<int>(f, "batch");
    c.sequence = number<int>(f, "sequence");
    c.hidden = number<int>(f, "hidden");
    c.intermediate = number<int>(f, "intermediate");
    c.query_heads = number<int>(f, "query_heads");
    c.kv_heads = number<int>(f, "kv_heads");
    c.head_dim = number<int>(f, "head_dim");
    c.rms_epsilon = number<float>(f, "rms_epsilon");
    c.rope_theta = number<float>(f, "rope_theta");
    c.causal = number<int>(f, "causal") != 0;
    const std::string& ffn = required(f, "ffn");
    if (ffn == decoder_ffn_name(DecoderFFNKind::Dense)) c.ffn = DecoderFFNKind::Dense;
    else if (ffn == decoder_ffn_name(DecoderFFNKind::MoE)) c.ffn = DecoderFFNKind::MoE;
    else throw std::runtime_error("unknown .sfe ffn: " + ffn);
    c.experts = number<int>(f, "experts");
    c.top_k = number<int>(f, "top_k");
    c.context_sequence = number<int>(f, "context_sequence");
    c.precision = parse_precision(required(f, "precision"));
    c.page_tokens = number<int>(f, "page_tokens");
    try {
        validate(c);
    } catch (const std::invalid_argument& e) {
        throw std::runtime_error(std::string(".sfe configuration: ") + e.what());
    }
    DecoderPlanPolicy& q = m.policy;
    q.weight_layout = number<int>(f, "weight_layout");
    if (q.weight_layout != SFG_LAYOUT_NK && q.weight_layout != SFG_LAYOUT_TILED)
        throw std::runtime_error("unknown .sfe weight layout");
    q.kv_splits = number<int>(f, "kv_splits");
    q.gemm_tile = number<int>(f, "gemm_tile");
    q.attn_waves = number<int>(f, "attn_waves");
    if (q.kv_splits < 0 || q.gemm_tile < SFG_TILE_AUTO || q.gemm_tile >= SFG_TILE_COUNT ||
        (q.attn_waves != 0 && q.attn_waves != 4 && q.attn_waves != 8))
        throw std::runtime_error("invalid .sfe plan policy");
    m.pages_per_seq = number<int>(f, "pages_per_seq");
    m.num_pages = number<int>(f, "num_pages");
    m.routing_trace = number<int>(f, "routing_trace") != 0;
    m.workspace_bytes = number<std::size_t>(f, "workspace_bytes");
    m.naive_bytes = number<std::size_t>(f, "naive_bytes");
    m.plan = parse_file("plan", required(f, "plan"));
    m.library = parse_file("library", required(f, "library"));
    m.constants = parse_file("constants", required(f, "constants"));
    const int objects = number<int>(f, "code_objects");
    if (objects <= 0 || objects > 64) throw std::runtime_error("invalid .sfe code object count");
    for (int i = 0; i < objects; ++i) {
        const std::string key = "code_object." + std::to_string(i);
        const std::string& v = required(f, key);
        const auto parts = split(v, ',');
        if (parts.size() != 4) throw std::runtime_error("malformed .sfe manifest field: " + key + "=" + v);
        DecoderPackageCodeObject co;
        co.file = parse_file(key, parts[0] + "," + parts[1] + "," + parts[2]);
        co.target_id = parts[3];
        if (co.target_id.find(std::string("--") + kTarget) == std::string::npos)
            throw std::runtime_error(".sfe code object for another target: " + co.target_id);
        m.code_objects.push_back(std::move(co));
    }
    const int buffers = number<int>(f, "buffers");
    if (buffers <= 0 || buffers > 256) throw std::runtime_error("invalid .sfe buffer count");
    std::size_t next = 0;
    for (int i = 0; i < buffers; ++i) {
        const std::string key = "buffer." + std::to_string(i);
        const std::string& v = required(f, key);
        const auto parts = split(v, ',');
        DecoderPackageBuffer b;
        try {
            if (parts.size() != 4 || parts[3].size() != 16) throw std::invalid_argument(v);
            b.name = parts[0];
            b.offset = std::stoull(parts[1]);
            b.bytes = std::stoull(parts[2]);
            b.checksum = parts[3];
        } catch (const std::exception&) {
            throw std::runtime_error("malformed .sfe manifest field: " + key + "=" + v);
        }
        if (b.bytes == 0 || b.offset < next || b.offset % kAlign != 0 || b.bytes > m.constants.bytes ||
            b.offset > m.constants.bytes - b.bytes)
            throw std::runtime_error(".sfe buffer " + b.name + " lies outside constants.bin");
        next = b.offset + b.bytes;
        m.buffers.push_back(std::move(b));
    }
    const int constants = number<int>(f, "constant_table");
    if (constants < 0 || constants > 256) throw std::runtime_error("invalid .sfe constant count");
    for (int i = 0; i < constants; ++i) {
        const std::string key = "constant." + std::to_string(i);
        m.constant_table.push_back(parse_constant(key, required(f, key)));
    }
    return m;
}

// ------------------------------------------------------------ save

DecoderPackageManifest save_decoder_package(const DecoderExecutablePlan& plan,
                                            const std::filesystem::path& path) {
    if (path.extension() != ".sfe") throw std::invalid_argument(".sfe package path must end in .sfe");
    if (!plan.device) throw std::invalid_argument("decoder plan was not compiled");
    auto& dev = *plan.device;

    const auto parent = path.parent_path().empty() ? std::filesystem::current_path() : path.parent_path();
    std::filesystem::create_directories(parent);
    const auto tmp = parent / (path.filename().string() + ".tmp-" + std::to_string(::getpid()));
    std::filesystem::remove_all(tmp);
    std::filesystem::create_directories(tmp / "kernels");
    try {
        DecoderPackageManifest m;
        m.schedforge_version = kVersion;
        m.abi = m.symbol = kAbi;
        m.target = kTarget;
        m.library_abi = dev.lib->abi_version();
        m.library_metadata = dev.lib->metadata();
        m.config = plan.config;
        m.policy = plan.policy;
        m.pages_per_seq = dev.desc.pages_per_seq;
        m.num_pages = dev.desc.num_pages;
        m.routing_trace = dev.desc.use_routing_trace != 0;
        m.workspace_bytes = plan.memory.workspace_bytes;
        m.naive_bytes = plan.memory.naive_bytes;
        m.constant_table = plan.constants;

        const std::string text = plan.dump();
        write_file(tmp / "plan.sfe", text.data(), text.size());
        m.plan = {"plan.sfe", text.size(), package_checksum(text.data(), text.size())};

        std::filesystem::copy_file(dev.lib->path, tmp / "libsfg_hip.so");
        m.library = describe_file(tmp, "libsfg_hip.so");
        const auto objects = embedded_code_objects(tmp / "libsfg_hip.so");
        for (std::size_t i = 0; i < objects.size(); ++i) {
            char name[64];
            std::snprintf(name, sizeof name, "kernels/%02zu.%s.hsaco", i, kTarget);
            write_file(tmp / name, objects[i].bytes.data(), objects[i].bytes.size());
            m.code_objects.push_back({{name, objects[i].bytes.size(),
                                       package_checksum(objects[i].bytes.data(), objects[i].bytes.size())},
                                      objects[i].target_id});
        }

        // Device buffers, in plan order, each at a 256-byte aligned offset.
        std::vector<std::pair<std::string, const DeviceBuffer*>> sources;
        for (const auto& [name, buffer] : dev.buffers) sources.emplace_back(name, &buffer);
        if (dev.trace_ids.ptr) {
            sources.emplace_back(kTraceIds, &dev.trace_ids);
            sources.emplace_back(kTraceWeights, &dev.trace_weights);
        }
        std::ofstream out(tmp / "constants.bin", std::ios::binary | std::ios::trunc);
        if (!out) throw std::runtime_error("cannot write .sfe package file: constants.bin");
        Fnv1a64 whole;
        std::size_t offset = 0;
        std::vector<char> host;
        {
            std::lock_guard lock(dev.mutex);
            hip_check(hipSetDevice(dev.ordinal), "hipSetDevice");
            for (const auto& [name, buffer] : sources) {
                const std::size_t pad = (kAlign - offset % kAlign) % kAlign;
                static const char zeros[kAlign] = {};
                out.write(zeros, static_cast<std::streamsize>(pad));
                whole.update(zeros, pad);
                offset += pad;
                host.resize(buffer->bytes);
                hip_check(hipMemcpyAsync(host.data(), buffer->ptr, buffer->bytes, hipMemcpyDeviceToHost,
                                         dev.stream),
                          "hipMemcpyAsync");
                dev.sync();
                out.write(host.data(), static_cast<std::streamsize>(buffer->bytes));
                whole.update(host.data(), buffer->bytes);
                m.buffers.push_back({name, offset, buffer->bytes, package_checksum(host.data(), buffer->bytes)});
                offset += buffer->bytes;
            }
        }
        out.close();
        if (!out) throw std::runtime_error("failed writing .sfe package file: constants.bin");
        m.constants = {"constants.bin", offset, whole.hex()};

        const std::string manifest = m.dump();
        write_file(tmp / "manifest.sfe", manifest.data(), manifest.size());
        std::filesystem::remove_all(path);
        std::filesystem::rename(tmp, path);
        return m;
    } catch (...) {
        std::filesystem::remove_all(tmp);
        throw;
    }
}

// ------------------------------------------------------------ inspect / load

DecoderPackageManifest inspect_decoder_package(const std::filesystem::path& path) {
    if (!std::filesystem::is_directory(path))
        throw std::runtime_error(".sfe package is not a directory: " + path.string());
    const auto m = DecoderPackageManifest::parse(read_file(path / "manifest.sfe"));
    auto check_file = [&](const DecoderPackageFile& f) {
        const std::string content = read_file(path / f.path);
        if (content.size() != f.bytes || package_checksum(content.data(), content.size()) != f.checksum)
            throw std::runtime_error(".sfe checksum mismatch: " + f.path);
    };
    check_file(m.plan);
    check_file(m.library);
    check_constants(path, m);
    for (const auto& co : m.code_objects) check_file(co.file);
    check_code_objects(path, m);

    // The packaged library's embedded metadata and entry point
    // (validate_embedded_metadata, aot_runtime.cpp:176-192).
    const auto lib = load_library(std::filesystem::absolute(path / m.library.path));
    if (lib->abi_version() != m.library_abi)
        throw std::runtime_error(".sfe embedded metadata mismatch: library_abi");
    if (m.library_metadata != lib->metadata())
        throw std::runtime_error(".sfe embedded metadata mismatch: library_metadata");
    if (!lib->lookup(m.symbol)) throw std::runtime_error(".sfe library lacks " + m.symbol);
    return m;
}

DecoderExecutablePlan load_decoder_package(const std::filesystem::path& path, int device) {
    const auto started = std::chrono::steady_clock::now();
    const auto m = inspect_decoder_package(path);

    DecoderExecutablePlan plan;
    plan.config = m.config;
    plan.constants = m.constant_table;
    plan.policy = m.policy;
    plan.device = std::make_unique<DecoderExecutablePlan::Device>();
    auto& dev = *plan.device;
    dev.lib = load_library(std::filesystem::absolute(path / m.library.path));
    dev.ordinal = device;
    plan.library_metadata = dev.lib->metadata();

    hipDeviceProp_t prop{};
    hip_check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    const std::string arch = prop.gcnArchName;
    if (arch != m.target && arch.rfind(m.target + ":", 0) != 0)
        throw std::runtime_error(".sfe target mismatch: package=" + m.target + " device=" + arch);
    hip_check(hipSetDevice(device), "hipSetDevice");
    hip_check(hipStreamCreate(&dev.stream), "hipStreamCreate");
    plan.hardware = describe_hardware(*dev.lib, device);

    // Buffers from constants.bin (checksums verified by inspect_decoder_package).
    std::ifstream in(path / m.constants.path, std::ios::binary);
    if (!in) throw std::runtime_error("cannot read .sfe package file: " + m.constants.path);
    std::vector<char> host;
    bool has_trace_ids = false, has_trace_weights = false;
    for (const auto& b : m.buffers) {
        host.resize(b.bytes);
        in.seekg(static_cast<std::streamoff>(b.offset));
        in.read(host.data(), static_cast<std::streamsize>(b.bytes));
        if (!in) throw std::runtime_error("cannot read .sfe buffer " + b.name);
        DeviceBuffer* target;
        if (b.name == kTraceIds) {
            dev.trace_ids = DeviceBuffer(b.bytes);
            target = &dev.trace_ids;
            has_trace_ids = true;
        } else if (b.name == kTraceWeights) {
            dev.trace_weights = DeviceBuffer(b.bytes);
            target = &dev.trace_weights;
            has_trace_weights = true;
        } else {
            for (const auto& [name, existing] : dev.buffers)
                if (name == b.name) throw std::runtime_error("duplicate .sfe plan buffer: " + b.name);
            dev.add(b.name, b.bytes);
            target = &dev.buffers.back().second;
            bind_buffer(dev.weights, b.name, target->ptr);
        }
        dev.upload(target->ptr, host.data(), b.bytes);
        dev.sync();  // `host` is reused by the next buffer
    }
    if (m.routing_trace != (has_trace_ids && has_trace_weights))
        throw std::runtime_error(".sfe routing trace buffers do not match the manifest");

    fill_layer_desc(dev.desc, m.config, m.policy, m.pages_per_seq, m.num_pages,
                    m.routing_trace);
    const std::size_t ws = allocate_workspace(dev);
    if (ws != m.workspace_bytes)
        throw std::runtime_error(".sfe workspace size differs from the packaged library's plan");
    plan.memory.workspace_bytes = ws;
    plan.memory.naive_bytes = m.naive_bytes;
    for (const auto& constant : plan.constants) plan.memory.constant_bytes += constant.bytes;
    plan.compile_milliseconds =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - started).count();
    return plan;
}

}  // namespace schedforge::hip
