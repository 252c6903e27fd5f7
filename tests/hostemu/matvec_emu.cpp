// matvec_emu.cpp - drives g3k_matvec (gemma3.c_amd/csrc/matvec.hip, built for
// the host against the emulation headers in this directory) on one case read
// from files, and writes what the kernel produced.  TEST INFRASTRUCTURE.
//
//   matvec_emu <dir>
//
// <dir>/args.txt: mode n_mat K M0 M1 M2 pre has_w_post has_w_next x_offset eps
// <dir>/*.bin inputs (raw little-endian): A0 / A1 / A2 bf16 [M][K]; x fp32 [K]
// (without pre); with pre: t, r fp32 [K] and w_post / w_next bf16 [K] when
// present.  x_offset > 0 places x that many floats into its allocation (an
// unaligned x).  Writes y0 .. y{n_out-1}.bin (fp32 [M]) and, with pre,
// r_out.bin.  Every buffer is its own heap allocation of exactly its size, so
// AddressSanitizer sees any access beyond it.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "g3k.h"

namespace {

template <typename T>
std::vector<T> read_bin(const std::string &path, size_t n, size_t lead = 0) {
    std::vector<T> v(lead + n);
    FILE *f = std::fopen(path.c_str(), "rb");
    if (!f || std::fread(v.data() + lead, sizeof(T), n, f) != n) {
        std::fprintf(stderr, "matvec_emu: cannot read %zu values from %s\n", n, path.c_str());
        std::exit(2);
    }
    std::fclose(f);
    return v;
}

void write_bin(const std::string &path, const float *p, size_t n) {
    FILE *f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(p, sizeof(float), n, f) != n) {
        std::fprintf(stderr, "matvec_emu: cannot write %s\n", path.c_str());
        std::exit(2);
    }
    std::fclose(f);
}

}  // namespace

int main(int argc, char **argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: matvec_emu <dir>\n");
        return 2;
    }
    const std::string dir = argv[1];
    int mode, n_mat, K, M[3], pre, has_wp, has_wn, x_off;
    float eps;
    FILE *f = std::fopen((dir + "/args.txt").c_str(), "r");
    if (!f || std::fscanf(f, "%d %d %d %d %d %d %d %d %d %d %f", &mode, &n_mat, &K, &M[0], &M[1], &M[2], &pre,
                          &has_wp, &has_wn, &x_off, &eps) != 11) {
        std::fprintf(stderr, "matvec_emu: bad args.txt\n");
        return 2;
    }
    std::fclose(f);
    std::vector<std::vector<uint16_t>> A(n_mat);
    for (int m = 0; m < n_mat; m++) A[m] = read_bin<uint16_t>(dir + "/A" + std::to_string(m) + ".bin", (size_t)M[m] * K);
    const int n_out = mode == G3K_MV_GEGLU ? 1 : n_mat;
    std::vector<std::vector<float>> y(n_out);
    for (int m = 0; m < n_out; m++) y[m].assign(M[m], -12345.0f);
    std::vector<float> x, t, r, r_out;
    std::vector<uint16_t> wp, wn;
    g3k_matvec_args a = {};
    a.K = K;
    a.n_mat = n_mat;
    a.mode = mode;
    for (int m = 0; m < n_mat; m++) {
        a.A[m] = A[m].data();
        a.M[m] = M[m];
        if (m < n_out) a.y[m] = y[m].data();
    }
    if (pre) {
        t = read_bin<float>(dir + "/t.bin", K);
        r = read_bin<float>(dir + "/r.bin", K);
        r_out.assign(K, -12345.0f);
        if (has_wp) wp = read_bin<uint16_t>(dir + "/w_post.bin", K);
        if (has_wn) wn = read_bin<uint16_t>(dir + "/w_next.bin", K);
        a.pre_t = t.data();
        a.pre_r = r.data();
        a.pre_r_out = r_out.data();
        a.pre_w_post = has_wp ? wp.data() : nullptr;
        a.pre_w_next = has_wn ? wn.data() : nullptr;
        a.pre_eps = eps;
    } else {
        x = read_bin<float>(dir + "/x.bin", K, (size_t)x_off);
        a.x = x.data() + x_off;
    }
    const int rc = g3k_matvec(&a, nullptr);
    if (rc) {
        std::fprintf(stderr, "matvec_emu: g3k_matvec returned %d\n", rc);
        return 1;
    }
    for (int m = 0; m < n_out; m++) write_bin(dir + "/y" + std::to_string(m) + ".bin", y[m].data(), y[m].size());
    if (pre) write_bin(dir + "/r_out.bin", r_out.data(), r_out.size());
    std::printf("matvec_emu: ok\n");
    return 0;
}
