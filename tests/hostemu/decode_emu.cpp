// decode_emu.cpp - drives g3k_decode (gemma3.c_amd/csrc/decode.hip, built for
// the host against the emulation headers in this directory) on one case read
// from files, and writes what the kernels produced.  TEST INFRASTRUCTURE.
//
//   decode_emu <dir>
//
// <dir>/args.txt: fused group n_kv n_heads cache_floats row_stride
//                 head_stride n_stream skip new_slot rows_per_split n_splits
//                 nt_loads has_norm has_mask eps qscale [xm_heads]
// (xm_heads > 0: the one-launch form with that many query heads per
// workgroup; the run checks that it leaves its arrival counters zero)
// <dir>/*.bin inputs (raw little-endian): q [H_q*D], k_new / v_new [H_kv*D]
// (fused), q_norm / k_norm bf16 [D] (has_norm), rope_row [D] (fused),
// kc / vc [cache_floats] (row r of head h at h*head_stride + r*row_stride),
// mask [n_stream] (has_mask).
// Writes out.bin [H_q*D], kc_out.bin and vc_out.bin.  Every buffer is its
// own heap allocation of exactly its size, so AddressSanitizer sees any
// access beyond it.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "g3k.h"

namespace {

template <typename T>
std::vector<T> read_bin(const std::string &path, size_t n) {
    std::vector<T> v(n);
    FILE *f = std::fopen(path.c_str(), "rb");
    if (!f || std::fread(v.data(), sizeof(T), n, f) != n) {
        std::fprintf(stderr, "decode_emu: cannot read %zu values from %s\n", n, path.c_str());
        std::exit(2);
    }
    std::fclose(f);
    return v;
}

template <typename T>
void write_bin(const std::string &path, const std::vector<T> &v) {
    FILE *f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(v.data(), sizeof(T), v.size(), f) != v.size()) {
        std::fprintf(stderr, "decode_emu: cannot write %s\n", path.c_str());
        std::exit(2);
    }
    std::fclose(f);
}

}  // namespace

int main(int argc, char **argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: decode_emu <dir>\n");
        return 2;
    }
    const std::string dir = argv[1];
    int fused, group, n_kv, n_heads, n_stream, skip, new_slot, rps, n_splits, nt_loads, has_norm, has_mask;
    long long cache, row_stride, head_stride;
    float eps, qscale;
    int xm_heads = 0;
    FILE *f = std::fopen((dir + "/args.txt").c_str(), "r");
    if (!f || std::fscanf(f, "%d %d %d %d %lld %lld %lld %d %d %d %d %d %d %d %d %f %f", &fused, &group, &n_kv,
                          &n_heads, &cache, &row_stride, &head_stride, &n_stream, &skip, &new_slot, &rps,
                          &n_splits, &nt_loads, &has_norm, &has_mask, &eps, &qscale) != 17) {
        std::fprintf(stderr, "decode_emu: bad args.txt\n");
        return 2;
    }
    if (std::fscanf(f, "%d", &xm_heads) != 1) xm_heads = 0;
    std::fclose(f);
    const size_t D = G3K_HEAD_DIM, qs = (size_t)n_heads * D, ks = (size_t)n_kv * D;

    std::vector<float> q = read_bin<float>(dir + "/q.bin", qs);
    std::vector<float> kc = read_bin<float>(dir + "/kc.bin", cache);
    std::vector<float> vc = read_bin<float>(dir + "/vc.bin", cache);
    std::vector<float> k_new, v_new, rope, mask;
    std::vector<uint16_t> qn, kn;
    if (fused) {
        k_new = read_bin<float>(dir + "/k_new.bin", ks);
        v_new = read_bin<float>(dir + "/v_new.bin", ks);
        rope = read_bin<float>(dir + "/rope_row.bin", D);
    }
    if (has_norm) {
        qn = read_bin<uint16_t>(dir + "/q_norm.bin", D);
        kn = read_bin<uint16_t>(dir + "/k_norm.bin", D);
    }
    if (has_mask) mask = read_bin<float>(dir + "/mask.bin", (size_t)n_stream);
    std::vector<float> out(qs, -12345.0f);
    std::vector<float> ws_acc((size_t)n_kv * G3K_MAX_SPLITS * group * D, -1.0f);
    std::vector<float> ws_ml((size_t)n_kv * G3K_MAX_SPLITS * group * 2, -1.0f);
    std::vector<unsigned> xcount(G3K_XM_COUNTERS(n_heads), 0u);

    g3k_decode_args a = {};
    a.q = q.data();
    a.k_new = fused ? k_new.data() : nullptr;
    a.v_new = fused ? v_new.data() : nullptr;
    a.q_norm = has_norm ? qn.data() : nullptr;
    a.k_norm = has_norm ? kn.data() : nullptr;
    a.rope_row = fused ? rope.data() : nullptr;
    a.eps = eps;
    a.kc = kc.data();
    a.vc = vc.data();
    a.row_stride = row_stride;
    a.head_stride = head_stride;
    a.n_stream = n_stream;
    a.skip = skip;
    a.new_slot = new_slot;
    a.mask = has_mask ? mask.data() : nullptr;
    a.qscale = qscale;
    a.rows_per_split = rps;
    a.n_splits = n_splits;
    a.n_kv_heads = n_kv;
    a.group = group;
    a.out = out.data();
    a.ws_acc = ws_acc.data();
    a.ws_ml = ws_ml.data();
    a.nt_loads = nt_loads;
    a.xm_heads = xm_heads;
    a.xm_count = xm_heads ? xcount.data() : nullptr;
    const int rc = g3k_decode(&a, fused, nullptr);
    if (rc) {
        std::fprintf(stderr, "decode_emu: g3k_decode returned %d\n", rc);
        return 1;
    }
    for (unsigned v : xcount)
        if (v) {
            std::fprintf(stderr, "decode_emu: an arrival counter was left at %u\n", v);
            return 1;
        }
    write_bin(dir + "/out.bin", out);
    write_bin(dir + "/kc_out.bin", kc);
    write_bin(dir + "/vc_out.bin", vc);
    std::printf("decode_emu: ok\n");
    return 0;
}
