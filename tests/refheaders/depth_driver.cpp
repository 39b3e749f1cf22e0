// depth_driver.cpp - runs the reference's RVQ depth decoder (src/depth-decoder.h
// with src/gguf-weights.h, src/weight-ctx.h, src/backend.h), compiled
// unchanged from the reference tree, on the MI355X ggml backend through this
// build's ggml API layer.  Test infrastructure: tests/test_gpu_refheaders.py
// writes the GGUF and the inputs, runs this program and checks its outputs.
//
//   depth_driver <depth.gguf> <io_dir> <n_frames>
//
// io_dir/single_seq.bin: f32 [8][4096] raw step embeddings; for S = 2..8 the
// first S rows go through DepthDecoder::forward (one cached graph per S,
// src/depth-decoder.h:247-285, :413-430), writing single_hiddens.bin (the
// S x 4096 normalised hidden states of every S, concatenated) and
// single_logits.bin ([7][1024], audio_heads[S - 2] on the last step).
// io_dir/frames.bin: per frame f32 seq_init [2][2][4096] (cond stream, then
// uncond), rand [7], cfg, top_k; each frame runs DepthDecoder::forward_frame
// (the fused 7-step CFG graph with in-graph sampling, src/depth-decoder.h:
// 294-411, :432-461) for one song, writing codes.bin (int32 [n_frames][7]),
// cond_hiddens.bin (f32 [n_frames][7][4096]) and step_logits.bin (f32
// [n_frames][7][2][1024], each step's cond / uncond head logits).  Prints one JSON line with
// the backend's graph statistics.
#include "depth-decoder.h"

#include "cpu_standin.h"

using namespace refdrv;

int main(int argc, char ** argv) {
    if (argc != 4) {
        fprintf(stderr, "usage: %s <depth.gguf> <io_dir> <n_frames>\n", argv[0]);
        return 2;
    }
    const std::string dir      = argv[2];
    const int         n_frames = atoi(argv[3]);
    register_cpu_standin();

    static DepthDecoder dd;
    if (!dd.load(argv[1])) {
        fprintf(stderr, "[driver] DepthDecoder::load failed\n");
        return 3;
    }
    const int DIM = DepthDecoder::DIM, V = DepthDecoder::VOCAB, NC = DepthDecoder::CODEBOOKS - 1;

    std::vector<float> seq = read_vec<float>(dir + "/single_seq.bin");
    if (seq.size() < (size_t) DepthDecoder::MAX_SEQ * DIM) {
        fprintf(stderr, "[driver] single_seq.bin too short\n");
        return 2;
    }
    std::vector<float> hid_all, logits_all((size_t) NC * V);
    for (int S = 2; S <= DepthDecoder::MAX_SEQ; S++) {
        std::vector<float> h((size_t) S * DIM);
        if (!dd.forward(seq.data(), S, h.data(), logits_all.data() + (size_t) (S - 2) * V)) {
            fprintf(stderr, "[driver] forward(S=%d) failed\n", S);
            return 4;
        }
        hid_all.insert(hid_all.end(), h.begin(), h.end());
    }
    write_bytes(dir + "/single_hiddens.bin", hid_all.data(), hid_all.size() * 4);
    write_bytes(dir + "/single_logits.bin", logits_all.data(), logits_all.size() * 4);

    // per frame: seq_init [2][2][DIM], rand [NC], cfg, top_k (as f32)
    std::vector<float>   fr  = read_vec<float>(dir + "/frames.bin");
    const size_t         per = (size_t) 4 * DIM + NC + 2;
    std::vector<int32_t> codes((size_t) n_frames * NC);
    std::vector<float>   ch((size_t) n_frames * NC * DIM);
    std::vector<float>   step_logits((size_t) n_frames * NC * V * 2);
    if (fr.size() < per * n_frames) {
        fprintf(stderr, "[driver] frames.bin too short\n");
        return 2;
    }
    for (int f = 0; f < n_frames; f++) {
        const float * p     = fr.data() + per * f;
        const float   cfg   = p[4 * DIM + NC];
        const int     top_k = (int) p[4 * DIM + NC + 1];
        std::vector<int> c(NC);
        if (!dd.forward_frame(p, p + 4 * DIM, cfg, top_k, 1, c.data(), ch.data() + (size_t) f * NC * DIM)) {
            fprintf(stderr, "[driver] forward_frame(%d) failed\n", f);
            return 5;
        }
        for (int i = 0; i < NC; i++) {
            codes[(size_t) f * NC + i] = c[(size_t) i];
        }
        // each step's head logits [V, 2] (cond, uncond): the MUL_MAT nodes of
        // audio_heads[cb - 1] in the frame graph (graph tensors keep their
        // memory after the compute)
        for (int cb = 1; cb <= NC; cb++) {
            ggml_tensor * lg = nullptr;
            for (int i = 0; i < ggml_graph_n_nodes(dd.fused.graph); i++) {
                ggml_tensor * n = ggml_graph_node(dd.fused.graph, i);
                if (n->op == GGML_OP_MUL_MAT && n->src[0] == dd.audio_heads[cb - 1]) {
                    lg = n;
                }
            }
            if (!lg || ggml_nbytes(lg) != (size_t) V * 2 * sizeof(float)) {
                fprintf(stderr, "[driver] no head logits node for codebook %d\n", cb);
                return 6;
            }
            ggml_backend_tensor_get(lg, step_logits.data() + ((size_t) f * NC + cb - 1) * V * 2, 0, ggml_nbytes(lg));
        }
    }
    write_bytes(dir + "/step_logits.bin", step_logits.data(), step_logits.size() * 4);
    write_bytes(dir + "/codes.bin", codes.data(), codes.size() * 4);
    write_bytes(dir + "/cond_hiddens.bin", ch.data(), ch.size() * 4);

    int64_t            replays = -1, eager = -1;
    ggml_backend_dev_t dev     = ggml_backend_get_device(dd.backend);
    ggml_backend_reg_t reg     = dev ? ggml_backend_dev_backend_reg(dev) : nullptr;
    if (reg) {
        auto stats = (void (*)(ggml_backend_t, int64_t *, int64_t *)) ggml_backend_reg_get_proc_address(
            reg, "ggml_backend_mi355x_graph_stats");
        if (stats) {
            stats(dd.backend, &replays, &eager);
        }
    }
    printf("{\"backend\": \"%s\", \"fused_nodes\": %d, \"replays\": %lld, \"eager\": %lld}\n",
           ggml_backend_name(dd.backend), dd.fused.graph ? ggml_graph_n_nodes(dd.fused.graph) : 0,
           (long long) replays, (long long) eager);
    fflush(stdout);
    dd.free();
    return 0;
}
