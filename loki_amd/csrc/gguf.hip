// gguf.hip -- the reference's model shards as this library reads them: a GGUF tensor index over one or more files and a
// loader that makes one MoE layer resident in HBM (the reference indexes its shards with ggml's gguf API and reads each
// expert at tensor offset + e * ggml_row_size(type, ne0) * ne1, src/server_core_fused.cpp:97-110, 295-305).
//
// GGUF (ggml's container, versions 2 and 3, little-endian), restated from its published specification:
//   u32 magic "GGUF", u32 version, u64 tensor count, u64 kv count;
//   kv: string key, u32 value type, value (0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array
//       {u32 type, u64 count, values}, 10 u64, 11 i64, 12 f64); string = u64 length + bytes;
//   tensor info: string name, u32 n_dims, u64 ne[n_dims], u32 ggml type, u64 offset (from the data section);
//   the data section starts at the next multiple of general.alignment (u32, default 32) after the infos.
// Expert tensors are [ne0 = columns, ne1 = rows, ne2 = experts], row-major, experts contiguous.
#include "fl_ctx.h"

#include <fcntl.h>
#include <unistd.h>

#include <map>

using namespace lk;

namespace {

// ggml types this index sizes (block elements, block bytes); others are indexed with nbytes = 0
struct TypeInfo { int blck; int bytes; int fl; };   // fl: the FL_* code, -1 when the library has no kernel for it
bool type_info(uint32_t t, TypeInfo & ti) {
    switch (t) {
        case 0: ti = { 1, 4, -1 }; return true;       // F32
        case 1: ti = { 1, 2, -1 }; return true;       // F16
        case 2: ti = { 32, 18, -1 }; return true;     // Q4_0
        case 3: ti = { 32, 20, -1 }; return true;     // Q4_1
        case 6: ti = { 32, 22, -1 }; return true;     // Q5_0
        case 7: ti = { 32, 24, -1 }; return true;     // Q5_1
        case 8: ti = { 32, 34, FL_Q80 }; return true; // Q8_0
        case 9: ti = { 32, 36, -1 }; return true;     // Q8_1
        case 10: ti = { 256, 84, FL_Q2K }; return true;
        case 11: ti = { 256, 110, FL_Q3K }; return true;
        case 12: ti = { 256, 144, FL_Q4K }; return true;
        case 13: ti = { 256, 176, FL_Q5K }; return true;
        case 14: ti = { 256, 210, FL_Q6K }; return true;
        case 15: ti = { 256, 292, -1 }; return true;  // Q8_K
        case 16: ti = { 256, 66, FL_IQ2 }; return true;   // IQ2_XXS
        case 17: ti = { 256, 74, -1 }; return true;   // IQ2_XS
        case 18: ti = { 256, 98, -1 }; return true;   // IQ3_XXS
        case 19: ti = { 256, 50, -1 }; return true;   // IQ1_S
        case 20: ti = { 32, 18, -1 }; return true;    // IQ4_NL
        case 21: ti = { 256, 110, -1 }; return true;  // IQ3_S
        case 22: ti = { 256, 82, -1 }; return true;   // IQ2_S
        case 23: ti = { 256, 136, -1 }; return true;  // IQ4_XS
        case 24: ti = { 1, 1, -1 }; return true;      // I8
        case 25: ti = { 1, 2, -1 }; return true;      // I16
        case 26: ti = { 1, 4, -1 }; return true;      // I32
        case 27: ti = { 1, 8, -1 }; return true;      // I64
        case 28: ti = { 1, 8, -1 }; return true;      // F64
        case 29: ti = { 256, 56, -1 }; return true;   // IQ1_M
        case 30: ti = { 1, 2, -1 }; return true;      // BF16
        default: return false;
    }
}

struct KV { uint32_t type = 0; uint64_t u = 0; int64_t i = 0; double f = 0; std::string s; uint64_t count = 0; };

// buffered sequential reader over a file descriptor with bounds checks
struct Reader {
    int fd; uint64_t pos = 0, size = 0;
    std::vector<uint8_t> buf; uint64_t bstart = 0, blen = 0;
    bool fill(uint64_t at, uint64_t need) {
        if (at >= bstart && at + need <= bstart + blen) { return true; }
        const uint64_t want = std::max<uint64_t>(need, 1 << 20);
        buf.resize(want);
        const ssize_t r = pread(fd, buf.data(), want, (off_t) at);
        if (r < (ssize_t) need) { return false; }
        bstart = at; blen = (uint64_t) r;
        return true;
    }
    bool get(void * dst, uint64_t n) {
        if (n > (1ull << 30) || pos + n > size || !fill(pos, n)) { return false; }
        std::memcpy(dst, buf.data() + (pos - bstart), n); pos += n;
        return true;
    }
    bool skip(uint64_t n) { if (pos + n > size) { return false; } pos += n; return true; }
    template <class T> bool num(T & v) { return get(&v, sizeof v); }
    bool str(std::string & s) {
        uint64_t n; if (!num(n) || n > (1ull << 24)) { return false; }
        s.resize(n); return n == 0 || get(&s[0], n);
    }
};

bool read_value(Reader & r, uint32_t type, KV & kv, int depth) {
    switch (type) {
        case 0: case 1: case 7: { uint8_t v; if (!r.num(v)) { return false; } kv.u = v; kv.i = type == 1 ? (int8_t) v : v; return true; }
        case 2: case 3: { uint16_t v; if (!r.num(v)) { return false; } kv.u = v; kv.i = type == 3 ? (int16_t) v : v; return true; }
        case 4: case 5: { uint32_t v; if (!r.num(v)) { return false; } kv.u = v; kv.i = type == 5 ? (int32_t) v : (int64_t) v; return true; }
        case 6: { float v; if (!r.num(v)) { return false; } kv.f = v; return true; }
        case 10: case 11: { uint64_t v; if (!r.num(v)) { return false; } kv.u = v; kv.i = (int64_t) v; return true; }
        case 12: { double v; if (!r.num(v)) { return false; } kv.f = v; return true; }
        case 8: return r.str(kv.s);
        case 9: {
            if (depth > 0) { return false; }
            uint32_t et; uint64_t n; if (!r.num(et) || !r.num(n)) { return false; }
            kv.count = n;
            static const int fixed[13] = { 1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8 };
            if (et > 12 || et == 9) { return false; }
            if (et == 8) { for (uint64_t k = 0; k < n; ++k) { std::string s; if (!r.str(s)) { return false; } } return true; }
            if (n > r.size) { return false; }
            return r.skip(n * (uint64_t) fixed[et]);
        }
        default: return false;
    }
}

}  // namespace

struct FLGguf {
    struct T { int file; uint32_t type; int n_dims; int64_t ne[4]; uint64_t offset; uint64_t nbytes; };
    std::vector<std::string> paths;
    std::vector<int> fds;
    std::vector<std::string> names;
    std::vector<T> tensors;
    std::map<std::string, int> by_name;
    std::map<std::string, KV> kv;   // first file's value wins
};

static void set_err(char * err, size_t len, const char * fmt, ...) {
    if (!err || len == 0) { return; }
    va_list ap; va_start(ap, fmt); std::vsnprintf(err, len, fmt, ap); va_end(ap);
}

extern "C" FLGguf * fl_gguf_open(const char * const * paths, int npaths, char * err, size_t errlen) {
    if (!paths || npaths <= 0) { set_err(err, errlen, "no files"); return nullptr; }
    FLGguf * g = new FLGguf();
    auto bad = [&](const char * why, int f) { set_err(err, errlen, "%s: %s", paths[f] ? paths[f] : "(null)", why); fl_gguf_close(g); return (FLGguf *) nullptr; };
    for (int f = 0; f < npaths; ++f) {
        if (!paths[f]) { return bad("null path", f); }
        const int fd = open(paths[f], O_RDONLY);
        if (fd < 0) { return bad("cannot open", f); }
        g->paths.push_back(paths[f]); g->fds.push_back(fd);
        Reader r; r.fd = fd; r.size = (uint64_t) lseek(fd, 0, SEEK_END);
        uint32_t magic, version; uint64_t nt, nkv;
        if (!r.num(magic) || magic != 0x46554747u) { return bad("not a GGUF file (magic)", f); }
        if (!r.num(version) || (version != 2 && version != 3)) { return bad("unsupported GGUF version (2 and 3 are read)", f); }
        if (!r.num(nt) || !r.num(nkv) || nt > (1u << 24) || nkv > (1u << 24)) { return bad("truncated header", f); }
        uint32_t align = 32;
        for (uint64_t k = 0; k < nkv; ++k) {
            std::string key; uint32_t type; KV v;
            if (!r.str(key) || !r.num(type)) { return bad("truncated metadata", f); }
            v.type = type;
            if (!read_value(r, type, v, 0)) { return bad("bad metadata value", f); }
            if (key == "general.alignment" && type == 4) {
                if (v.u == 0 || (v.u & (v.u - 1))) { return bad("general.alignment is not a power of two", f); }
                align = (uint32_t) v.u;
            }
            if (!g->kv.count(key)) { g->kv[key] = v; }
        }
        std::vector<FLGguf::T> local; std::vector<std::string> lnames;
        for (uint64_t k = 0; k < nt; ++k) {
            std::string name; uint32_t nd;
            if (!r.str(name) || !r.num(nd) || nd == 0 || nd > 4) { return bad("bad tensor info", f); }
            FLGguf::T t{}; t.file = f; t.n_dims = (int) nd;
            for (int d = 0; d < 4; ++d) { t.ne[d] = 1; }
            for (uint32_t d = 0; d < nd; ++d) { uint64_t v; if (!r.num(v) || v > (1ull << 40)) { return bad("bad tensor dims", f); } t.ne[d] = (int64_t) v; }
            if (!r.num(t.type) || !r.num(t.offset)) { return bad("truncated tensor info", f); }
            TypeInfo ti;
            if (type_info(t.type, ti)) {
                if (t.ne[0] % ti.blck) { return bad("tensor row not a whole number of blocks", f); }
                // the size as a checked product: a wrapped value would skip the end-of-file test below
                uint64_t nb = (uint64_t) (t.ne[0] / ti.blck);
                bool ovf = __builtin_mul_overflow(nb, (uint64_t) ti.bytes, &nb);
                for (int d = 1; d < 4; ++d) { ovf = ovf || __builtin_mul_overflow(nb, (uint64_t) t.ne[d], &nb); }
                if (ovf) { return bad("tensor size overflows 64 bits", f); }
                t.nbytes = nb;
            }
            if (t.offset % align) { return bad("tensor offset not aligned", f); }
            local.push_back(t); lnames.push_back(name);
        }
        const uint64_t data0 = (r.pos + align - 1) / align * align;
        for (size_t k = 0; k < local.size(); ++k) {
            FLGguf::T t = local[k];
            uint64_t end = 0;
            if (__builtin_add_overflow(t.offset, data0, &t.offset) || __builtin_add_overflow(t.offset, t.nbytes, &end) || end > r.size) {
                return bad("tensor data past the end of the file", f);
            }
            auto it = g->by_name.find(lnames[k]);
            if (it != g->by_name.end()) { g->tensors[it->second] = t; continue; }   // a later file's tensor replaces it (eng:105)
            g->by_name[lnames[k]] = (int) g->tensors.size();
            g->tensors.push_back(t); g->names.push_back(lnames[k]);
        }
    }
    return g;
}

extern "C" void fl_gguf_close(FLGguf * g) {
    if (!g) { return; }
    for (int fd : g->fds) { close(fd); }
    delete g;
}

extern "C" int fl_gguf_n_tensors(const FLGguf * g) { return g ? (int) g->tensors.size() : 0; }
extern "C" const char * fl_gguf_tensor_name(const FLGguf * g, int i) {
    return (g && i >= 0 && i < (int) g->names.size()) ? g->names[i].c_str() : nullptr;
}

static void fill_tensor(const FLGguf::T & t, FLGgufTensor * out) {
    out->file = t.file; out->type = (int) t.type; out->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) { out->ne[d] = t.ne[d]; }
    out->offset = t.offset; out->nbytes = t.nbytes;
    TypeInfo ti;
    out->fl_format = type_info(t.type, ti) ? ti.fl : -1;
    out->row_bytes = type_info(t.type, ti) ? (uint64_t) (t.ne[0] / ti.blck) * (uint64_t) ti.bytes : 0;
}

extern "C" int fl_gguf_tensor(const FLGguf * g, const char * name, FLGgufTensor * out) {
    if (!g || !name || !out) { return FL_EINVAL; }
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) { return FL_ERANGE; }
    fill_tensor(g->tensors[it->second], out);
    return FL_OK;
}

extern "C" int fl_gguf_tensor_at(const FLGguf * g, int i, FLGgufTensor * out) {
    if (!g || !out || i < 0 || i >= (int) g->tensors.size()) { return FL_EINVAL; }
    fill_tensor(g->tensors[i], out);
    return FL_OK;
}

extern "C" int fl_gguf_get_int(const FLGguf * g, const char * key, int64_t * out) {
    if (!g || !key || !out) { return FL_EINVAL; }
    auto it = g->kv.find(key);
    if (it == g->kv.end()) { return FL_ERANGE; }
    const uint32_t t = it->second.type;
    if (t > 5 && t != 7 && t != 10 && t != 11) { return FL_EINVAL; }
    *out = it->second.i;
    return FL_OK;
}
extern "C" int fl_gguf_get_float(const FLGguf * g, const char * key, double * out) {
    if (!g || !key || !out) { return FL_EINVAL; }
    auto it = g->kv.find(key);
    if (it == g->kv.end()) { return FL_ERANGE; }
    if (it->second.type != 6 && it->second.type != 12) { return FL_EINVAL; }
    *out = it->second.f;
    return FL_OK;
}
extern "C" const char * fl_gguf_get_str(const FLGguf * g, const char * key) {
    if (!g || !key) { return nullptr; }
    auto it = g->kv.find(key);
    return (it == g->kv.end() || it->second.type != 8) ? nullptr : it->second.s.c_str();
}

extern "C" int fl_gguf_read(const FLGguf * g, const FLGgufTensor * t, uint64_t off, uint64_t bytes, void * dst) {
    if (!g || !t || !dst || t->file < 0 || t->file >= (int) g->fds.size()) { return FL_EINVAL; }
    if (off > t->nbytes || bytes > t->nbytes - off) { return FL_ERANGE; }
    uint8_t * p = static_cast<uint8_t *>(dst); uint64_t done = 0;
    while (done < bytes) {
        const ssize_t r = pread(g->fds[t->file], p + done, (size_t) std::min<uint64_t>(bytes - done, 1ull << 30), (off_t) (t->offset + off + done));
        if (r <= 0) { return FL_EINVAL; }
        done += (uint64_t) r;
    }
    return FL_OK;
}

// ---------------------------------------------------------------- one MoE layer resident in HBM
// two pinned staging buffers and their events, allocated once per layer load
struct Staging {
    static constexpr size_t CH = 32u << 20;
    uint8_t * hb[2] = { nullptr, nullptr }; hipEvent_t ev[2] = { nullptr, nullptr };
    int init(FLCtx * c) {
        for (int k = 0; k < 2; ++k) {
            if (hipHostMalloc((void **) &hb[k], CH, hipHostMallocDefault) != hipSuccess) { hb[k] = nullptr; return fail(c, FL_ENOMEM, "pinned staging"); }
            if (hipEventCreateWithFlags(&ev[k], hipEventDisableTiming) != hipSuccess) { ev[k] = nullptr; return fail(c, FL_EHIP, "event"); }
        }
        return FL_OK;
    }
    ~Staging() { for (int k = 0; k < 2; ++k) { if (ev[k]) { (void) hipEventDestroy(ev[k]); } if (hb[k]) { (void) hipHostFree(hb[k]); } } }
};

// file bytes of a tensor -> device memory through the staging buffers (the read of one chunk overlaps the copy of the
// previous one); waits for its copies before returning
static int upload(FLCtx * c, const FLGguf * g, Staging & sg, const FLGgufTensor & t, uint8_t * dst) {
    constexpr size_t CH = Staging::CH;
    uint8_t * const * hb = sg.hb; hipEvent_t * ev = sg.ev;
    int rc = FL_OK;
    for (uint64_t off = 0, k = 0; rc == FL_OK && off < t.nbytes; off += CH, ++k) {
        const size_t n = (size_t) std::min<uint64_t>(CH, t.nbytes - off);
        const int b = (int) (k & 1);
        if (k >= 2 && hipEventSynchronize(ev[b]) != hipSuccess) { rc = fail(c, FL_EHIP, "staging wait"); break; }
        if (fl_gguf_read(g, &t, off, n, hb[b]) != FL_OK) { rc = fail(c, FL_EINVAL, "read of %s failed", g->paths[t.file].c_str()); break; }
        if (hipMemcpyAsync(dst + off, hb[b], n, hipMemcpyHostToDevice, c->st) != hipSuccess || hipEventRecord(ev[b], c->st) != hipSuccess) {
            rc = fail(c, FL_EHIP, "upload copy"); break;
        }
    }
    if (hipStreamSynchronize(c->st) != hipSuccess && rc == FL_OK) { rc = fail(c, FL_EHIP, "upload sync"); }
    return rc;
}

extern "C" int fl_gguf_load_moe_layer(FLCtx * c, const FLGguf * g, int layer, int layout, FLGgufLayer * out) {
    if (!c) { return FL_EINVAL; }
    if (!g || !out || layer < 0) { return fail(c, FL_EINVAL, "null index / output or negative layer"); }
    if (layout != FL_LAYOUT_GGML && layout != FL_LAYOUT_TILED) { return fail(c, FL_EINVAL, "layout %d", layout); }
    std::memset(out, 0, sizeof *out);
    const std::string p = "blk." + std::to_string(layer) + ".";
    FLGgufTensor tr{}, tb{}, tn{}, te[3]{}, ts[3]{};
    bool r16 = false;
    if (fl_gguf_tensor(g, (p + "ffn_gate_inp.weight").c_str(), &tr) != FL_OK) {
        if (fl_gguf_tensor(g, (p + "ffn_gate_inp_f16.weight").c_str(), &tr) != FL_OK) { return fail(c, FL_ERANGE, "%sffn_gate_inp.weight: no such tensor (not a MoE layer?)", p.c_str()); }
        r16 = true;
    }
    const char * en[3] = { "ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight" };
    const char * sn[3] = { "ffn_gate_shexp.weight", "ffn_up_shexp.weight", "ffn_down_shexp.weight" };
    if (fl_gguf_tensor(g, (p + "exp_probs_b.bias").c_str(), &tb) != FL_OK) { return fail(c, FL_ERANGE, "%sexp_probs_b.bias: no such tensor", p.c_str()); }
    for (int k = 0; k < 3; ++k) {
        if (fl_gguf_tensor(g, (p + en[k]).c_str(), &te[k]) != FL_OK) { return fail(c, FL_ERANGE, "%s%s: no such tensor", p.c_str(), en[k]); }
        if (fl_gguf_tensor(g, (p + sn[k]).c_str(), &ts[k]) != FL_OK) { return fail(c, FL_ERANGE, "%s%s: no such tensor", p.c_str(), sn[k]); }
    }
    const bool has_norm = fl_gguf_tensor(g, (p + "ffn_norm.weight").c_str(), &tn) == FL_OK;
    // shapes: gate/up [E, H, n_exp], down [H, E, n_exp], shared [E, H] / [H, E], router [E, n_exp], bias [n_exp]
    const int64_t E = te[0].ne[0], H = te[0].ne[1], ne = te[0].ne[2];
    auto shp = [](const FLGgufTensor & t, int64_t a, int64_t b, int64_t cc) { return t.ne[0] == a && t.ne[1] == b && t.ne[2] == cc && t.ne[3] == 1; };
    if (!shp(te[1], E, H, ne) || !shp(te[2], H, E, ne) || !shp(ts[0], E, H, 1) || !shp(ts[1], E, H, 1) || !shp(ts[2], H, E, 1) ||
        !shp(tr, E, ne, 1) || !shp(tb, ne, 1, 1) || (has_norm && !shp(tn, E, 1, 1))) {
        return fail(c, FL_EINVAL, "%s: tensor shapes do not form one MoE layer (E %lld, H %lld, experts %lld)", p.c_str(), (long long) E, (long long) H, (long long) ne);
    }
    if (tr.type != (r16 ? 1 : 0) || tb.type != 0 || (has_norm && tn.type != 0)) { return fail(c, FL_EINVAL, "%s: router, bias and norm must be F32 (router F16 as ffn_gate_inp_f16)", p.c_str()); }
    if (ne <= 0 || ne > 256 || E <= 0 || H <= 0 || E > 65536 || H > 65536 || E % 1024 || H % 1024) { return fail(c, FL_EINVAL, "%s: %lld experts, E %lld, H %lld (experts <= 256, E and H positive multiples of 1024 up to 65536)", p.c_str(), (long long) ne, (long long) E, (long long) H); }
    int fm[6];
    for (int k = 0; k < 3; ++k) { fm[k] = te[k].fl_format; fm[3 + k] = ts[k].fl_format; }
    if (fm[0] != FL_IQ2 || fm[1] != FL_IQ2) { return fail(c, FL_ESCOPE, "%s: routed gate/up must be IQ2_XXS (types %d, %d)", p.c_str(), te[0].type, te[1].type); }
    if (fm[2] != FL_IQ2 && fm[2] != FL_Q2K && fm[2] != FL_Q3K) { return fail(c, FL_ESCOPE, "%s: routed down type %d (IQ2_XXS, Q2_K or Q3_K)", p.c_str(), te[2].type); }
    for (int k = 3; k < 6; ++k) {
        if (fm[k] != FL_IQ2 && kq_block_bytes(fm[k]) == 0) { return fail(c, FL_ESCOPE, "%s: shared-expert type %d (IQ2_XXS or Q2_K / Q3_K / Q5_K / Q6_K)", p.c_str(), ts[k - 3].type); }
    }
    if ((fm[3] == FL_IQ2) != (fm[4] == FL_IQ2)) { return fail(c, FL_ESCOPE, "%s: shared gate and up must both be IQ2_XXS or both K-quants", p.c_str()); }
    // one allocation: router (F32), bias, norm, 3 routed tensors, 3 shared matrices; 256-byte aligned parts
    auto al = [](uint64_t v) { return (v + 255) / 256 * 256; };
    const uint64_t szr = (uint64_t) E * ne * 4, szb = (uint64_t) ne * 4, szn = has_norm ? (uint64_t) E * 4 : 0;
    uint64_t off[9], tot = 0;
    const uint64_t parts[9] = { szr, szb, szn, te[0].nbytes, te[1].nbytes, te[2].nbytes, ts[0].nbytes, ts[1].nbytes, ts[2].nbytes };
    for (int k = 0; k < 9; ++k) { off[k] = tot; tot += al(parts[k]); }
    uint8_t * mem = nullptr;
    if (hipMalloc((void **) &mem, tot) != hipSuccess) { (void) hipGetLastError(); return fail(c, FL_ENOMEM, "device allocation of %llu bytes", (unsigned long long) tot); }
    uint8_t * stage = nullptr;   // ggml-layout staging for the tiled layout, and for the F16 router
    uint64_t stage_sz = r16 ? tr.nbytes : 0;
    if (layout == FL_LAYOUT_TILED) {
        for (int k = 0; k < 3; ++k) {
            if (fm[k] == FL_IQ2) { stage_sz = std::max(stage_sz, te[k].nbytes); }
            if (fm[3 + k] == FL_IQ2) { stage_sz = std::max(stage_sz, ts[k].nbytes); }
        }
    }
    Staging sg;
    int rc = sg.init(c);
    if (rc == FL_OK && stage_sz && hipMalloc((void **) &stage, stage_sz) != hipSuccess) { (void) hipGetLastError(); rc = fail(c, FL_ENOMEM, "staging allocation"); }
    if (rc == FL_OK) {
        if (r16) {
            rc = upload(c, g, sg, tr, stage);
            if (rc == FL_OK && launch_f16_to_f32((const uint16_t *) stage, (float *) (mem + off[0]), E * ne, c->st) != hipSuccess) { rc = fail(c, FL_EHIP, "router widening"); }
        } else {
            rc = upload(c, g, sg, tr, mem + off[0]);
        }
    }
    if (rc == FL_OK) { rc = upload(c, g, sg, tb, mem + off[1]); }
    if (rc == FL_OK && has_norm) { rc = upload(c, g, sg, tn, mem + off[2]); }
    const FLGgufTensor * mats[6] = { &te[0], &te[1], &te[2], &ts[0], &ts[1], &ts[2] };
    for (int k = 0; k < 6 && rc == FL_OK; ++k) {
        uint8_t * dst = mem + off[3 + k];
        const FLGgufTensor & t = *mats[k];
        if (layout == FL_LAYOUT_TILED && fm[k] == FL_IQ2) {   // K-quant matrices stay as stored in either layout
            rc = upload(c, g, sg, t, stage);
            const int R = (int) t.ne[1], K = (int) t.ne[0], nm = (int) t.ne[2];
            const size_t ms = (size_t) t.row_bytes * (size_t) R;
            if (rc == FL_OK && launch_pack_tiled(stage, ms, dst, ms, R, K, nm, c->st) != hipSuccess) { rc = fail(c, FL_EHIP, "tiled packing"); }
            if (rc == FL_OK && hipStreamSynchronize(c->st) != hipSuccess) { rc = fail(c, FL_EHIP, "packing sync"); }
        } else {
            rc = upload(c, g, sg, t, dst);
        }
    }
    if (stage) { (void) hipStreamSynchronize(c->st); (void) hipFree(stage); }
    if (rc != FL_OK) { (void) hipFree(mem); std::memset(out, 0, sizeof *out); return rc; }
    FLMoeLayer & L = out->L;
    L.gate_inp = (const float *) (mem + off[0]); L.probs_b = (const float *) (mem + off[1]);
    L.gate_exps = mem + off[3]; L.up_exps = mem + off[4]; L.down_exps = mem + off[5];
    L.sh_gate = mem + off[6]; L.sh_up = mem + off[7]; L.sh_down = mem + off[8];
    L.layout = layout; L.n_exp = (int) ne; L.E = (int) E; L.H = (int) H;
    out->ffn_norm = has_norm ? (const float *) (mem + off[2]) : nullptr;
    out->fmt_down = fm[2]; out->fmt_sh_gate = fm[3]; out->fmt_sh_up = fm[4]; out->fmt_sh_down = fm[5];
    out->expert_stride[0] = te[0].row_bytes * (uint64_t) H; out->expert_stride[1] = te[1].row_bytes * (uint64_t) H;
    out->expert_stride[2] = te[2].row_bytes * (uint64_t) E;
    out->mem = mem; out->bytes = tot;
    if (layout == FL_LAYOUT_TILED) {   // the tiled IQ2_XXS matrices are read in place by fl_moe / fl_wide_moe / fl_ffn_begin
        for (int k = 0; k < 6; ++k) { if (fm[k] == FL_IQ2) { tiled_add(mem + off[3 + k], mats[k]->nbytes); } }
    }
    return FL_OK;
}

extern "C" void fl_gguf_free_layer(FLGgufLayer * l) {
    if (!l) { return; }
    if (l->mem) { tiled_remove_within(l->mem, l->bytes); (void) hipDeviceSynchronize(); (void) hipFree(l->mem); }
    std::memset(l, 0, sizeof *l);
}
