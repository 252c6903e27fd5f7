// attn_emu.cpp - runs a script of g3attn C-ABI calls against the whole
// library (gemma3.c_amd/host + csrc) built for the emulated GPU of
// hip/hip_runtime.h, under AddressSanitizer + UndefinedBehaviorSanitizer.
// TEST INFRASTRUCTURE.
//
//   attn_emu <dir>
//
// <dir>/script.txt holds one call per line; file names are relative to <dir>
// (raw little-endian arrays; "-" for an absent optional one).  Any nonzero
// return stops the run with exit status 1 and the library's error text.
//
//   create H Hkv max_context window num_layers eps rope_local rope_global
//          [hidden intermediate vocab]
//   kv_write layer slot n k v                  (rows [n][Hkv][256])
//   kv_read layer slot n k_out v_out
//   prefill layer start_pos n Q K V q_norm k_norm out
//   prefill_device ...                          (same, device pointers)
//   decode layer pos q k v q_norm k_norm out
//   matmul N M K W X C                          (g3attn_matmul_bf16_device)
//   gqa H Hkv seq q k v mask|- out [head_dim]   (g3attn_gqa, host pointers;
//                                                head_dim 256 if absent, scale
//                                                1 / sqrt(head_dim))
//   gqa_noalloc H Hkv seq q k v mask|- out      (device copies, null stream;
//                                                fails if the call allocates)
//   matvec M K A x y                            (g3attn_matvec_bf16, host)
//   matvec_device M K A x y                     (g3attn_matvec_bf16_device)
//   kv_append layer start n K V k_norm|-
//   layer_attention layer pos hidden x wq wk wv wo q_norm|- k_norm|- out
//   model prefix     the model's bf16 tensors from prefix + "embed.bin",
//                    "norm.bin" and "L<l>_<tensor>.bin" (a missing file is a
//                    NULL tensor), kept in host memory and as device copies
//   upload                                      (g3attn_upload_weights, host)
//   forward_device token pos logits|-           (the device copies)
//   forward_token token pos logits              (the uploaded model)
//   prefill_tokens n tokens start logits        (the uploaded model)
//   destroy
//   front_stage_only Hkv nk V vt_out            (g3k_rope_write_stage with an
//                    empty batch, ra.n = 0, and no cache: the V^T staging of
//                    nk keys alone; vt_out gets the bf16 hi plane [Hkv][256][ldk])
//
// At the end it prints "launch <kernel> <launches> <workgroups> <threads> <ms>" for every
// kernel launched and "attn_emu: ok".
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "g3attn.h"
#include "g3k.h"

namespace {

const char *const kLayerTensors[13] = {
    "input_layernorm", "q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm",
    "post_attention_layernorm", "gate_proj", "up_proj", "down_proj", "pre_feedforward_layernorm",
    "post_feedforward_layernorm"};

std::string g_dir;

[[noreturn]] void die(const std::string &what) {
    std::fprintf(stderr, "attn_emu: %s\n", what.c_str());
    std::exit(2);
}

template <typename T>
std::vector<T> read_bin(const std::string &name, size_t n) {
    std::vector<T> v(n);
    FILE *f = std::fopen((g_dir + "/" + name).c_str(), "rb");
    if (!f || std::fread(v.data(), sizeof(T), n, f) != n) die("cannot read " + std::to_string(n) + " values from " + name);
    std::fclose(f);
    return v;
}

template <typename T>
void write_bin(const std::string &name, const T *p, size_t n) {
    FILE *f = std::fopen((g_dir + "/" + name).c_str(), "wb");
    if (!f || std::fwrite(p, sizeof(T), n, f) != n) die("cannot write " + name);
    std::fclose(f);
}

// An optional bf16 row of 256 gains: "-" is NULL.
struct Gain {
    std::vector<uint16_t> v;
    const uint16_t *ptr() const { return v.empty() ? nullptr : v.data(); }
};
Gain read_gain(const std::string &name) {
    Gain g;
    if (name != "-") g.v = read_bin<uint16_t>(name, 256);
    return g;
}

// A device copy of a host array (emulated device memory: its own heap block).
template <typename T>
T *to_device(const std::vector<T> &h) {
    void *d = nullptr;
    if (hipMalloc(&d, h.size() * sizeof(T)) != hipSuccess) die("hipMalloc");
    hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice);
    return static_cast<T *>(d);
}

bool exists(const std::string &name) {
    FILE *f = std::fopen((g_dir + "/" + name).c_str(), "rb");
    if (f) std::fclose(f);
    return f != nullptr;
}

size_t file_elems(const std::string &name, size_t elem) {
    FILE *f = std::fopen((g_dir + "/" + name).c_str(), "rb");
    if (!f) die("cannot open " + name);
    std::fseek(f, 0, SEEK_END);
    const long n = std::ftell(f);
    std::fclose(f);
    return (size_t)n / elem;
}

// A model's tensors: host arrays (for g3attn_upload_weights) and device
// copies (for g3attn_forward_device), in g3attn_weights structs.
struct Model {
    std::vector<std::vector<uint16_t>> host;
    std::vector<void *> dev;
    g3attn_weights h{}, d{};
    const uint16_t *load(const std::string &name, const uint16_t **dev_slot) {
        if (!exists(name)) {
            *dev_slot = nullptr;
            return nullptr;
        }
        host.push_back(read_bin<uint16_t>(name, file_elems(name, 2)));
        void *p = nullptr;
        if (hipMalloc(&p, host.back().size() * 2) != hipSuccess) die("hipMalloc");
        hipMemcpy(p, host.back().data(), host.back().size() * 2, hipMemcpyHostToDevice);
        dev.push_back(p);
        *dev_slot = static_cast<const uint16_t *>(p);
        return host.back().data();
    }
    ~Model() {
        for (void *p : dev) hipFree(p);
    }
};

void check(int rc, const std::string &call) {
    if (rc) {
        std::fprintf(stderr, "attn_emu: %s returned %d: %s\n", call.c_str(), rc, g3attn_last_error());
        std::exit(1);
    }
}

}  // namespace

int main(int argc, char **argv) {
    if (argc != 2) die("usage: attn_emu <dir>");
    g_dir = argv[1];
    std::ifstream script(g_dir + "/script.txt");
    if (!script) die("no script.txt");
    g3attn_ctx *ctx = nullptr;
    int H = 0, Hkv = 0, layers = 0, hidden = 0, vocab = 0;
    Model *model = nullptr;
    const size_t D = 256;
    std::string line;
    while (std::getline(script, line)) {
        std::istringstream in(line);
        std::string cmd;
        if (!(in >> cmd) || cmd[0] == '#') continue;
        if (cmd == "create") {
            int max_ctx, window, inter = 0;
            float eps;
            std::string rl, rg;
            in >> H >> Hkv >> max_ctx >> window >> layers >> eps >> rl >> rg;
            if (!in) die("bad create line");
            if (!(in >> hidden >> inter >> vocab)) hidden = inter = vocab = 0;
            g3attn_config cfg;
            g3attn_default_config(&cfg);
            cfg.num_heads = H;
            cfg.num_kv_heads = Hkv;
            cfg.max_context = max_ctx;
            cfg.sliding_window = window;
            cfg.num_layers = layers;
            cfg.rmsnorm_eps = eps;
            if (hidden) {
                cfg.hidden_size = hidden;
                cfg.intermediate_size = inter;
                cfg.vocab_size = vocab;
            }
            const auto tl = read_bin<float>(rl, (size_t)max_ctx * D);
            const auto tg = read_bin<float>(rg, (size_t)max_ctx * D);
            ctx = g3attn_create(&cfg, max_ctx, tl.data(), tg.data());
            if (!ctx) {
                std::fprintf(stderr, "attn_emu: g3attn_create failed: %s\n", g3attn_last_error());
                return 1;
            }
        } else if (cmd == "kv_write" || cmd == "kv_read") {
            int layer, slot, n;
            std::string kf, vf;
            in >> layer >> slot >> n >> kf >> vf;
            if (!in || !ctx) die("bad " + cmd + " line");
            const size_t cnt = (size_t)n * Hkv * D;
            if (cmd == "kv_write") {
                const auto k = read_bin<float>(kf, cnt), v = read_bin<float>(vf, cnt);
                check(g3attn_kv_write(ctx, layer, slot, n, k.data(), v.data()), cmd);
            } else {
                std::vector<float> k(cnt), v(cnt);
                check(g3attn_kv_read(ctx, layer, slot, n, k.data(), v.data()), cmd);
                write_bin(kf, k.data(), cnt);
                write_bin(vf, v.data(), cnt);
            }
        } else if (cmd == "prefill" || cmd == "prefill_device") {
            int layer, start, n;
            std::string qf, kf, vf, qn, kn, of;
            in >> layer >> start >> n >> qf >> kf >> vf >> qn >> kn >> of;
            if (!in || !ctx) die("bad prefill line");
            const auto Q = read_bin<float>(qf, (size_t)n * H * D);
            const auto K = read_bin<float>(kf, (size_t)n * Hkv * D);
            const auto V = read_bin<float>(vf, (size_t)n * Hkv * D);
            const Gain gq = read_gain(qn), gk = read_gain(kn);
            std::vector<float> out((size_t)n * H * D, -12345.0f);
            if (cmd == "prefill") {
                check(g3attn_prefill(ctx, layer, start, n, Q.data(), K.data(), V.data(), gq.ptr(), gk.ptr(),
                                     out.data()),
                      cmd);
            } else {
                float *dQ = to_device(Q), *dK = to_device(K), *dV = to_device(V), *dO = to_device(out);
                uint16_t *dq = gq.v.empty() ? nullptr : to_device(gq.v);
                uint16_t *dk = gk.v.empty() ? nullptr : to_device(gk.v);
                check(g3attn_prefill_device(ctx, layer, start, n, dQ, dK, dV, dq, dk, dO), cmd);
                check(g3attn_synchronize(ctx), "g3attn_synchronize");
                hipMemcpy(out.data(), dO, out.size() * sizeof(float), hipMemcpyDeviceToHost);
                for (void *p : {(void *)dQ, (void *)dK, (void *)dV, (void *)dO, (void *)dq, (void *)dk}) hipFree(p);
            }
            write_bin(of, out.data(), out.size());
        } else if (cmd == "decode") {
            int layer, pos;
            std::string qf, kf, vf, qn, kn, of;
            in >> layer >> pos >> qf >> kf >> vf >> qn >> kn >> of;
            if (!in || !ctx) die("bad decode line");
            const auto q = read_bin<float>(qf, (size_t)H * D);
            const auto k = read_bin<float>(kf, (size_t)Hkv * D);
            const auto v = read_bin<float>(vf, (size_t)Hkv * D);
            const Gain gq = read_gain(qn), gk = read_gain(kn);
            std::vector<float> out((size_t)H * D, -12345.0f);
            check(g3attn_decode(ctx, layer, pos, q.data(), k.data(), v.data(), gq.ptr(), gk.ptr(), out.data()), cmd);
            write_bin(of, out.data(), out.size());
        } else if (cmd == "matmul") {
            int N, M, K;
            std::string wf, xf, cf;
            in >> N >> M >> K >> wf >> xf >> cf;
            if (!in || !ctx) die("bad matmul line");
            const auto W = read_bin<uint16_t>(wf, (size_t)M * K);
            const auto X = read_bin<float>(xf, (size_t)N * K);
            std::vector<float> C((size_t)N * M, -12345.0f);
            uint16_t *dW = to_device(W);
            float *dX = to_device(X), *dC = to_device(C);
            check(g3attn_matmul_bf16_device(ctx, dC, dW, dX, N, M, K), cmd);
            check(g3attn_synchronize(ctx), "g3attn_synchronize");
            hipMemcpy(C.data(), dC, C.size() * sizeof(float), hipMemcpyDeviceToHost);
            hipFree(dW);
            hipFree(dX);
            hipFree(dC);
            write_bin(cf, C.data(), C.size());
        } else if (cmd == "gqa" || cmd == "gqa_noalloc") {
            int h, hkv, seq, hd = (int)D;
            std::string qf, kf, vf, mf, of;
            in >> h >> hkv >> seq >> qf >> kf >> vf >> mf >> of;
            if (!in) die("bad " + cmd + " line");
            if (!(in >> hd)) hd = (int)D;   // optional head_dim
            const auto q = read_bin<float>(qf, (size_t)h * hd);
            const auto k = read_bin<float>(kf, (size_t)seq * hkv * hd);
            const auto v = read_bin<float>(vf, (size_t)seq * hkv * hd);
            std::vector<float> mask;
            if (mf != "-") mask = read_bin<float>(mf, (size_t)seq);
            std::vector<float> out((size_t)h * hd, -12345.0f);
            const float scale = 1.0f / std::sqrt((float)hd);
            if (cmd == "gqa") {
                g3attn_gqa(out.data(), q.data(), k.data(), v.data(), h, hkv, seq, hd, scale,
                           mask.empty() ? nullptr : mask.data(), nullptr);
                if (out[0] == -12345.0f) check(-1, cmd);   // g3attn_gqa reports failure only by leaving out as is
            } else {
                float *dq = to_device(q), *dk = to_device(k), *dv = to_device(v), *dout = to_device(out);
                float *dm = mask.empty() ? nullptr : to_device(mask);
                // the entry point allocates and frees nothing (its split
                // partials live in the library's fixed device scratch)
                const unsigned long long allocs = hostemu_alloc_calls();
                check(g3attn_gqa_noalloc(dout, dq, dk, dv, h, hkv, seq, hd, scale, dm, nullptr), cmd);
                if (hostemu_alloc_calls() != allocs) die("gqa_noalloc called an allocating entry point");
                hipDeviceSynchronize();
                hipMemcpy(out.data(), dout, out.size() * sizeof(float), hipMemcpyDeviceToHost);
                for (void *p : {(void *)dq, (void *)dk, (void *)dv, (void *)dout, (void *)dm}) hipFree(p);
            }
            write_bin(of, out.data(), out.size());
        } else if (cmd == "matvec" || cmd == "matvec_device") {
            int M, K;
            std::string af, xf, yf;
            in >> M >> K >> af >> xf >> yf;
            if (!in) die("bad " + cmd + " line");
            const auto A = read_bin<uint16_t>(af, (size_t)M * K);
            const auto x = read_bin<float>(xf, (size_t)K);
            std::vector<float> y((size_t)M, -12345.0f);
            if (cmd == "matvec") {
                g3attn_matvec_bf16(y.data(), A.data(), x.data(), M, K, nullptr);
                if (M > 0 && y[0] == -12345.0f) check(-1, cmd);
            } else {
                if (!ctx) die("matvec_device needs a context");
                uint16_t *dA = to_device(A);
                float *dx = to_device(x), *dy = to_device(y);
                check(g3attn_matvec_bf16_device(ctx, dy, dA, dx, M, K), cmd);
                check(g3attn_synchronize(ctx), "g3attn_synchronize");
                hipMemcpy(y.data(), dy, y.size() * sizeof(float), hipMemcpyDeviceToHost);
                for (void *p : {(void *)dA, (void *)dx, (void *)dy}) hipFree(p);
            }
            write_bin(yf, y.data(), y.size());
        } else if (cmd == "kv_append") {
            int layer, start, n;
            std::string kf, vf, kn;
            in >> layer >> start >> n >> kf >> vf >> kn;
            if (!in || !ctx) die("bad kv_append line");
            const auto K = read_bin<float>(kf, (size_t)n * Hkv * D);
            const auto V = read_bin<float>(vf, (size_t)n * Hkv * D);
            const Gain gk = read_gain(kn);
            check(g3attn_kv_append(ctx, layer, start, n, K.data(), V.data(), gk.ptr()), cmd);
        } else if (cmd == "layer_attention") {
            int layer, pos, hid;
            std::string xf, wqf, wkf, wvf, wof, qn, kn, of;
            in >> layer >> pos >> hid >> xf >> wqf >> wkf >> wvf >> wof >> qn >> kn >> of;
            if (!in || !ctx) die("bad layer_attention line");
            const size_t qs = (size_t)H * D, ks = (size_t)Hkv * D;
            const auto x = read_bin<float>(xf, (size_t)hid);
            const auto wq = read_bin<uint16_t>(wqf, qs * hid), wk = read_bin<uint16_t>(wkf, ks * hid);
            const auto wv = read_bin<uint16_t>(wvf, ks * hid), wo = read_bin<uint16_t>(wof, hid * qs);
            const Gain gq = read_gain(qn), gk = read_gain(kn);
            std::vector<float> out((size_t)hid, -12345.0f);
            float *dx = to_device(x), *dout = to_device(out);
            uint16_t *dq = to_device(wq), *dk = to_device(wk), *dv = to_device(wv), *dw = to_device(wo);
            uint16_t *dqn = gq.v.empty() ? nullptr : to_device(gq.v);
            uint16_t *dkn = gk.v.empty() ? nullptr : to_device(gk.v);
            check(g3attn_layer_attention_device(ctx, layer, pos, dx, dq, dk, dv, dw, dqn, dkn, dout), cmd);
            check(g3attn_synchronize(ctx), "g3attn_synchronize");
            hipMemcpy(out.data(), dout, out.size() * sizeof(float), hipMemcpyDeviceToHost);
            for (void *p : {(void *)dx, (void *)dout, (void *)dq, (void *)dk, (void *)dv, (void *)dw, (void *)dqn,
                            (void *)dkn})
                hipFree(p);
            write_bin(of, out.data(), out.size());
        } else if (cmd == "model") {
            std::string prefix;
            in >> prefix;
            if (!in || model) die("bad model line");
            model = new Model;
            model->h.embed_tokens = model->load(prefix + "embed.bin", &model->d.embed_tokens);
            model->h.norm = model->load(prefix + "norm.bin", &model->d.norm);
            for (int l = 0; l < layers; l++) {
                const uint16_t **hs = reinterpret_cast<const uint16_t **>(&model->h.layers[l]);
                const uint16_t **ds = reinterpret_cast<const uint16_t **>(&model->d.layers[l]);
                for (int t = 0; t < 13; t++)
                    hs[t] = model->load(prefix + "L" + std::to_string(l) + "_" + kLayerTensors[t] + ".bin", &ds[t]);
            }
        } else if (cmd == "upload") {
            if (!ctx || !model) die("upload needs a context and a model");
            check(g3attn_upload_weights(ctx, &model->h), cmd);
        } else if (cmd == "forward_device" || cmd == "forward_token") {
            int token, pos;
            std::string lf;
            in >> token >> pos >> lf;
            if (!in || !ctx || !model) die("bad " + cmd + " line");
            std::vector<float> logits((size_t)vocab, -12345.0f);
            if (cmd == "forward_token") {
                check(g3attn_forward_token(ctx, token, pos, logits.data(), 1), cmd);
            } else {
                float *dl = lf == "-" ? nullptr : to_device(logits);
                check(g3attn_forward_device(ctx, &model->d, token, pos, dl, dl != nullptr, nullptr), cmd);
                check(g3attn_synchronize(ctx), "g3attn_synchronize");
                if (dl) hipMemcpy(logits.data(), dl, logits.size() * sizeof(float), hipMemcpyDeviceToHost);
                hipFree(dl);
            }
            if (lf != "-") write_bin(lf, logits.data(), logits.size());
        } else if (cmd == "prefill_tokens") {
            int n, start;
            std::string tf, lf;
            in >> n >> tf >> start >> lf;
            if (!in || !ctx || !model) die("bad prefill_tokens line");
            const auto tokens = read_bin<int>(tf, (size_t)n);
            std::vector<float> logits((size_t)vocab, -12345.0f);
            check(g3attn_prefill_tokens(ctx, tokens.data(), n, start, logits.data()), cmd);
            write_bin(lf, logits.data(), logits.size());
        } else if (cmd == "front_stage_only") {
            // The front launch with no batch tokens must stage V^T and touch
            // nothing of the (absent) cache destination.
            int hkv, nk;
            std::string vf, of;
            in >> hkv >> nk >> vf >> of;
            if (!in || hkv < 1 || nk < 1) die("bad front_stage_only line");
            const long long ldk = (nk + 63) / 64 * 64;
            const auto V = read_bin<float>(vf, (size_t)nk * hkv * D);
            float *dV = to_device(V);
            std::vector<uint16_t> zero((size_t)hkv * D * ldk, 0), zk((size_t)hkv * ldk * 2 * D, 0);
            uint16_t *dvt = to_device(zero), *dvl = to_device(zero), *dkq = to_device(zk);
            std::vector<int> flag(1, 0);
            int *dflag = to_device(flag);
            g3k_rope_write_args ra;
            std::memset(&ra, 0, sizeof ra);
            ra.n = 0;
            ra.n_kv_heads = hkv;
            ra.V = dV;   // k_dst / v_dst stay NULL
            g3k_stage_args sa;
            std::memset(&sa, 0, sizeof sa);
            sa.v_src = dV;
            sa.head_stride = D;
            sa.row_stride = (long long)hkv * D;
            sa.kk0 = 0;
            sa.cnt = (int)ldk;
            sa.nk = nk;
            sa.n_kv_heads = hkv;
            sa.kq = dkq;
            sa.vt = dvt;
            sa.vt_lo = dvl;
            sa.ldk = ldk;
            sa.v_lo_flag = dflag;
            sa.epoch = 1;
            const int rc = g3k_rope_write_stage(&ra, &sa, nullptr);
            if (rc) die("g3k_rope_write_stage returned " + std::to_string(rc));
            std::vector<uint16_t> vt(zero.size());
            hipMemcpy(vt.data(), dvt, vt.size() * sizeof(uint16_t), hipMemcpyDeviceToHost);
            write_bin(of, vt.data(), vt.size());
            for (void *p : {(void *)dV, (void *)dvt, (void *)dvl, (void *)dkq, (void *)dflag}) hipFree(p);
        } else if (cmd == "destroy") {
            g3attn_destroy(ctx);
            ctx = nullptr;
        } else {
            die("unknown command " + cmd);
        }
    }
    if (ctx) g3attn_destroy(ctx);
    delete model;
    hostemu_print_launches();
    std::printf("attn_emu: ok\n");
    return 0;
}
