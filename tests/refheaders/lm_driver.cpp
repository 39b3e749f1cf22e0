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

#include "cpu_standin.h"

using namespace refdrv;

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
