// lm_driver.cpp - runs the reference's Qwen3 LM code (src/qwen3-lm.h with
// src/qwen3-enc.h, src/gguf-weights.h, src/weight-ctx.h, src/backend.h,
// src/static-graph.h, src/graph-arena.h), compiled unchanged from the
// reference tree, on the MI355X ggml backend through this build's ggml API
// layer.  Test infrastructure: tests/test_gpu_refheaders.py writes a GGUF
// model and the inputs, runs this program and checks what it writes.
//
//   lm_driver <model.gguf> <io_dir> <n_steps> <max_seq>
//
// io_dir/tokens0.bin, tokens1.bin (int32 prompt tokens of the two CFG sets),
// io_dir/embeds.bin (f32 [n_steps][2][H] decode input embeddings).  Writes
// weights.bin (every loaded weight read back, GGUF bytes), prefill_logits.bin [2][V] and prefill_hidden.bin [2][H] (qw3lm_forward per
// set, src/qwen3-lm.h:451-643), kv.bin (every layer's f16 K then V cache
// after the prefill), decode_logits.bin [n_steps][2][V] and
// decode_hidden.bin [n_steps][2][H] (qw3lm_forward_batch, src/qwen3-lm.h:
// 645-934, on sets {0, 1} from the embeddings), and prints one JSON line with
// the backend's graph statistics.
#include "qwen3-lm.h"

#include "ggml-backend-impl.h"

#include <stdint.h>

#include <fstream>
#include <string>
#include <vector>

namespace {

// A CPU device for the reference's backend_init (src/backend.h:37-50,
// :135-146, which exits without one).  It runs nothing: supports_op is false
// for every op, so the scheduler places every graph on the MI355X backend.
// Its buffers are plain host memory.
struct host_buf {
    std::vector<uint8_t> bytes;
};

void hb_free(ggml_backend_buffer_t b) {
    delete (host_buf *) b->context;
}
void * hb_base(ggml_backend_buffer_t b) {
    return ((host_buf *) b->context)->bytes.data();
}
void hb_memset(ggml_backend_buffer_t, ggml_tensor * t, uint8_t v, size_t off, size_t n) {
    memset((char *) t->data + off, v, n);
}
void hb_set(ggml_backend_buffer_t, ggml_tensor * t, const void * d, size_t off, size_t n) {
    memcpy((char *) t->data + off, d, n);
}
void hb_get(ggml_backend_buffer_t, const ggml_tensor * t, void * d, size_t off, size_t n) {
    memcpy(d, (const char *) t->data + off, n);
}
void hb_clear(ggml_backend_buffer_t b, uint8_t v) {
    std::vector<uint8_t> & x = ((host_buf *) b->context)->bytes;
    memset(x.data(), v, x.size());
}
const ggml_backend_buffer_i k_hb_iface = { hb_free, hb_base, nullptr, hb_memset, hb_set, hb_get, nullptr, hb_clear,
                                           nullptr };

const char * hbt_name(ggml_backend_buffer_type_t) {
    return "CPU";
}
ggml_backend_buffer_t hbt_alloc(ggml_backend_buffer_type_t t, size_t size) {
    auto * h = new host_buf();
    h->bytes.resize(size + 64);
    return ggml_backend_buffer_init(t, k_hb_iface, h, size);
}
size_t hbt_align(ggml_backend_buffer_type_t) {
    return 64;
}
bool hbt_is_host(ggml_backend_buffer_type_t) {
    return true;
}

const char * cb_name(ggml_backend_t) {
    return "CPU";
}
void cb_free(ggml_backend_t b) {
    delete b;
}
void cb_sync(ggml_backend_t) {}
ggml_status cb_compute(ggml_backend_t, ggml_cgraph *) {
    fprintf(stderr, "[driver] the CPU stand-in was asked to compute a graph\n");
    return GGML_STATUS_FAILED;
}
ggml_guid k_cpu_guid = { { 'c', 'p', 'u', '-', 's', 't', 'a', 'n', 'd', '-', 'i', 'n', 0, 0, 0, 1 } };
const ggml_backend_i k_cb_iface = { cb_name, cb_free, nullptr, nullptr, nullptr, cb_sync, nullptr,
                                    nullptr, nullptr, nullptr, cb_compute, nullptr, nullptr, nullptr };

ggml_backend_buffer_type g_host_buft;
ggml_backend_device      g_cpu_dev;
ggml_backend_reg         g_cpu_reg;

const char * cd_name(ggml_backend_dev_t) {
    return "CPU";
}
const char * cd_desc(ggml_backend_dev_t) {
    return "host stand-in (runs no ops)";
}
void cd_mem(ggml_backend_dev_t, size_t * f, size_t * t) {
    *f = 0;
    *t = 0;
}
enum ggml_backend_dev_type cd_type(ggml_backend_dev_t) {
    return GGML_BACKEND_DEVICE_TYPE_CPU;
}
void cd_props(ggml_backend_dev_t d, ggml_backend_dev_props * p) {
    p->name        = cd_name(d);
    p->description = cd_desc(d);
    p->memory_free = p->memory_total = 0;
    p->type        = GGML_BACKEND_DEVICE_TYPE_CPU;
    p->device_id   = nullptr;
    p->caps        = { false, false, false, false };
}
ggml_backend_t cd_init(ggml_backend_dev_t d, const char *) {
    return new ggml_backend{ &k_cpu_guid, k_cb_iface, d, nullptr };
}
ggml_backend_buffer_type_t cd_buft(ggml_backend_dev_t) {
    return &g_host_buft;
}
bool cd_supports_op(ggml_backend_dev_t, const ggml_tensor *) {
    return false;
}
bool cd_supports_buft(ggml_backend_dev_t, ggml_backend_buffer_type_t t) {
    return ggml_backend_buft_is_host(t);
}
const ggml_backend_device_i k_cd_iface = { cd_name, cd_desc, cd_mem,         cd_type,          cd_props, cd_init,
                                           cd_buft, nullptr, nullptr,        cd_supports_op,   cd_supports_buft,
                                           nullptr, nullptr, nullptr,        nullptr };

const char * cr_name(ggml_backend_reg_t) {
    return "CPU";
}
size_t cr_count(ggml_backend_reg_t) {
    return 1;
}
ggml_backend_dev_t cr_dev(ggml_backend_reg_t, size_t i) {
    return i == 0 ? &g_cpu_dev : nullptr;
}
void set_n_threads(ggml_backend_t, int) {}
void * cr_proc(ggml_backend_reg_t, const char * name) {
    return strcmp(name, "ggml_backend_set_n_threads") == 0 ? (void *) set_n_threads : nullptr;
}
const ggml_backend_reg_i k_cr_iface = { cr_name, cr_count, cr_dev, cr_proc };

void register_cpu_standin() {
    g_host_buft = { { hbt_name, hbt_alloc, hbt_align, nullptr, nullptr, hbt_is_host }, &g_cpu_dev, nullptr };
    g_cpu_reg   = { GGML_BACKEND_API_VERSION, k_cr_iface, nullptr };
    g_cpu_dev   = { k_cd_iface, &g_cpu_reg, nullptr };
    ggml_backend_register(&g_cpu_reg);
}

template <typename T> std::vector<T> read_vec(const std::string & path) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) {
        fprintf(stderr, "[driver] cannot read %s\n", path.c_str());
        exit(2);
    }
    const size_t n = (size_t) f.tellg();
    f.seekg(0);
    std::vector<T> v(n / sizeof(T));
    f.read((char *) v.data(), (std::streamsize) (v.size() * sizeof(T)));
    return v;
}

void write_bytes(const std::string & path, const void * p, size_t n) {
    std::ofstream f(path, std::ios::binary);
    f.write((const char *) p, (std::streamsize) n);
    if (!f) {
        fprintf(stderr, "[driver] cannot write %s\n", path.c_str());
        exit(2);
    }
}

}  // namespace

int main(int argc, char ** argv) {
    if (argc != 5) {
        fprintf(stderr, "usage: %s <model.gguf> <io_dir> <n_steps> <max_seq>\n", argv[0]);
        return 2;
    }
    const std::string dir     = argv[2];
    const int         n_steps = atoi(argv[3]);
    const int         max_seq = atoi(argv[4]);
    register_cpu_standin();

    static Qwen3LM m;  // large (fixed arrays of tensors per set and layer)
    if (!qw3lm_load(&m, argv[1], max_seq, 2)) {
        fprintf(stderr, "[driver] qw3lm_load failed\n");
        return 3;
    }
    const int H = m.cfg.hidden_size, V = m.cfg.vocab_size;

    // every weight read back through ggml_backend_tensor_get (GGUF bytes):
    // embeddings, head, final norm, then per layer the tensors of
    // qwen3_load_layer (src/qwen3-enc.h:119-166) in declaration order
    {
        std::vector<ggml_tensor *> ws = { m.embed_tokens, m.lm_head, m.final_norm };
        for (int l = 0; l < m.cfg.n_layers; l++) {
            const Qwen3Layer & ly = m.layers[l];
            for (ggml_tensor * t : { ly.input_layernorm, ly.post_attn_layernorm, ly.qkv, ly.o_proj, ly.q_norm,
                                     ly.k_norm, ly.gate_up, ly.down_proj }) {
                ws.push_back(t);
            }
        }
        std::vector<uint8_t> wb;
        for (ggml_tensor * t : ws) {
            if (!t) {
                fprintf(stderr, "[driver] a weight expected by the test was not loaded (fused layout?)\n");
                return 4;
            }
            const size_t n = ggml_nbytes(t), o = wb.size();
            wb.resize(o + n);
            ggml_backend_tensor_get(t, wb.data() + o, 0, n);
        }
        write_bytes(dir + "/weights.bin", wb.data(), wb.size());
    }

    // prefill of each CFG set from its prompt tokens
    std::vector<float> logits((size_t) 2 * V), hidden((size_t) 2 * H);
    for (int s = 0; s < 2; s++) {
        std::vector<int32_t> tok = read_vec<int32_t>(dir + "/tokens" + std::to_string(s) + ".bin");
        std::vector<int>     ids(tok.begin(), tok.end());
        qw3lm_forward(&m, ids.data(), (int) ids.size(), s, logits.data() + (size_t) s * V, nullptr,
                      hidden.data() + (size_t) s * H);
    }
    write_bytes(dir + "/prefill_logits.bin", logits.data(), logits.size() * 4);
    write_bytes(dir + "/prefill_hidden.bin", hidden.data(), hidden.size() * 4);

    // the caches the decode starts from
    {
        std::vector<uint8_t> kv;
        for (int l = 0; l < m.cfg.n_layers; l++) {
            for (ggml_tensor * t : { m.kv_k4[l], m.kv_v4[l] }) {
                const size_t n = ggml_nbytes(t), o = kv.size();
                kv.resize(o + n);
                ggml_backend_tensor_get(t, kv.data() + o, 0, n);
            }
        }
        write_bytes(dir + "/kv.bin", kv.data(), kv.size());
    }

    // batched CFG decode from input embeddings (the frame feedback path)
    std::vector<float> emb = read_vec<float>(dir + "/embeds.bin");
    if (emb.size() < (size_t) n_steps * 2 * H) {
        fprintf(stderr, "[driver] embeds.bin too short\n");
        return 2;
    }
    std::vector<float> dl((size_t) n_steps * 2 * V), dh((size_t) n_steps * 2 * H);
    const int          sets[2] = { 0, 1 };
    for (int step = 0; step < n_steps; step++) {
        qw3lm_forward_batch(&m, nullptr, sets, 2, dl.data() + (size_t) step * 2 * V, 0, 0,
                            emb.data() + (size_t) step * 2 * H, dh.data() + (size_t) step * 2 * H);
    }
    write_bytes(dir + "/decode_logits.bin", dl.data(), dl.size() * 4);
    write_bytes(dir + "/decode_hidden.bin", dh.data(), dh.size() * 4);

    int64_t replays = -1, eager = -1;
    ggml_backend_dev_t dev = ggml_backend_get_device(m.backend);
    ggml_backend_reg_t reg = dev ? ggml_backend_dev_backend_reg(dev) : nullptr;
    if (reg) {
        auto stats = (void (*)(ggml_backend_t, int64_t *, int64_t *)) ggml_backend_reg_get_proc_address(
            reg, "ggml_backend_mi355x_graph_stats");
        if (stats) {
            stats(m.backend, &replays, &eager);
        }
    }
    printf("{\"backend\": \"%s\", \"direct_decode\": %s, \"kv_pos\": [%d, %d], \"replays\": %lld, \"eager\": %lld}\n",
           ggml_backend_name(m.backend), m.batch_graph.graph.direct ? "true" : "false", m.kv_pos[0], m.kv_pos[1],
           (long long) replays, (long long) eager);
    fflush(stdout);
    qw3lm_free(&m);
    return 0;
}
