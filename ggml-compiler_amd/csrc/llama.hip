// llama.hip - a Llama-style causal LM (GQA attention, SwiGLU FFN, RMSNorm, NEOX RoPE, f16 KV cache,
// Q4_0 or Q8_0 weights) executed with libgcq's kernels: the program ggml-compiler's causal_lm
// builds (ggml_compiler/llm.py:361-444) with its three entry points:
//   prefill(tokens, positions, mask) -> logits of the last token       (llm.py:12-13)
//   decode(token, position, mask1)   -> logits                          (llm.py:14)
//   generate(first, start)           -> greedy tokens, on the device    (llm.py:421-436)
// The KV cache is state, zeroed at creation and by reset (runtime/src/ggml_compiler_rt.cpp:528,
// :1020-1031). Per layer the graph is the one causal_lm emits at O3 (rms_norm, mul, mul_mat q/k/v,
// rope, set_rows, flash_attn, mul_mat o, add, rms_norm, mul, mul_mat gate/up, swiglu, mul_mat
// down, add; tests/unit/test_llm.py:130-134), with q/k/v and gate/up each one row-stacked weight
// (rows are independent, so the results equal separate mul_mats) and ten launches per layer.
//
// The decode step is captured once in a HIP graph (the counterpart of the reference's CUDA
// graphs, runtime/CMakeLists.txt:29-31). Its kernels read the token, position and KV length
// from a small device state that the step's last kernel advances, so a greedy generate is a run
// of graph launches with no host round trip.
#include "gcq_common.h"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/gcq.h"

namespace gcq {

void launch_encode(int type, const float * src, int64_t nrows, int64_t k, void * dst, hipStream_t s);
void launch_pack(int type, const void * src, int64_t nrows, int64_t k, void * dst, hipStream_t s);
void launch_unpack(int type, const void * src, int64_t nrows, int64_t k, void * dst, hipStream_t s);
void launch_gemv(int type, const void * w, int64_t N, int64_t K, const void * act, int64_t B, float * y, int64_t ldy,
                 hipStream_t s, const float * res);
void launch_gemm(int type, const void * w, int64_t N, int64_t K, const void * act, int64_t M, float * y, int64_t ldy,
                 hipStream_t s, const float * res);
void launch_get_rows(int type, const void * tab, int64_t nrows_tab, int64_t D, const int32_t * idx, int64_t n,
                     float * out, hipStream_t s);
void launch_fill_normal(float * dst, int64_t n, uint64_t seed, uint64_t offset, float stddev, hipStream_t s);
void launch_attn_split(const float * q, int64_t q_h, int64_t q_s, const void * k, int64_t k_h, int64_t k_j,
                       const void * v, int64_t v_h, int64_t v_j, const void * mask, int64_t m_s, int D, int Sq, int H,
                       int Hkv, int n_kv, float scale, float * po, float2 * pml, const AttnPlan & p,
                       const int * n_kv_dev, hipStream_t s);
void launch_rmsnorm_q8(const float * x, int64_t ldx, const float * w, float eps, int64_t rows, int64_t n, void * act,
                       hipStream_t s);
void launch_swiglu_q8(const float * g, const float * u, int64_t ld, int64_t n, int64_t rows, void * act,
                      hipStream_t s);
void launch_rope_kv(float * qkv, int64_t ld, const int32_t * pos, int S, int H, int Hkv, int D, float base,
                    void * cache, int64_t ctx, hipStream_t s);
void launch_merge_q8(const float * part_o, const float2 * part_ml, int nsplit, int Sq, int H, int D, float * out,
                     void * act, hipStream_t s);
void launch_causal_mask(void * mask, int S, int n_kv, int pos0, hipStream_t s);
void launch_move_rows(const void * src, void * dst, const int32_t * map, int64_t rows, int64_t row_bytes, bool scatter,
                      hipStream_t s);
void launch_scatter_cols(const float * src, int64_t lds, float * dst, int64_t ldd, const int32_t * map, int S, int n,
                         hipStream_t s);
AttnPlan attn_plan_decode(int D, int H, int G, int max_ctx, int max_split);
bool attn_decode_fits(int D, int G);
void launch_attn_decode(const float * q, int64_t q_h, const void * k, int64_t k_h, int64_t k_j, const void * v,
                        int64_t v_h, int64_t v_j, int D, int H, int Hkv, int n_kv, const int * n_kv_dev, float scale,
                        int nsplit, int chunk, int kv_rows, int GS, float * out, float * part_o, float2 * part_ml,
                        hipStream_t s, const Prefetch * pf, const void * mask, int nw_lanes);
int decode_group(int GT, int max_kv);
void launch_embed_rope(int type, const void * tab, int64_t nrows, int64_t D, const int32_t * idx, float * x,
                       const int32_t * pos, int head_dim, float base, void * cs, hipStream_t s);
void launch_step_end(const float * logits, int n, void * state, int32_t * out_tokens, int max_out, void * part,
                     void * counter, hipStream_t s);

int cu_count();

struct StepStateHost {
    int pos, n_kv, token, step;
};

namespace {

struct DevBuf {
    void * p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    explicit DevBuf(size_t bytes) : n(bytes) { check_hip(hipMalloc(&p, std::max<size_t>(bytes, 256)), "hipMalloc"); }
    DevBuf(const DevBuf &) = delete;
    DevBuf & operator=(const DevBuf &) = delete;
    DevBuf(DevBuf && o) noexcept : p(o.p), n(o.n) { o.p = nullptr; }
    DevBuf & operator=(DevBuf && o) noexcept {
        std::swap(p, o.p);
        std::swap(n, o.n);
        return *this;
    }
    ~DevBuf() {
        if (p) (void) hipFree(p);
    }
    template <class T> T * as() const { return reinterpret_cast<T *>(p); }
};

struct Tensor {
    std::string name;
    int type;           // T_F32 (norm weights) or the model's weight type
    int64_t rows, cols;
    bool random;        // drawn by init_random
    DevBuf buf;         // packed (quantized) or f32
    DevBuf perm;        // packed row r holds the weight's row perm[r] (int32); empty: same order
};

}  // namespace

struct Llama {
    gcq_llama_config c{};
    int max_prompt = 0;
    hipStream_t stream = nullptr;
    std::vector<Tensor> tensors;
    // indices into tensors
    int t_embd = -1, t_out_norm = -1, t_out = -1;
    struct Layer {
        int attn_norm, qkv, wo, ffn_norm, gate_up, down;
    };
    std::vector<Layer> layers;

    int64_t qkv_dim = 0, attn_dim = 0;
    DevBuf kv, x, qkv, gu, act_a, act_b, part_o, part_ml, mask, positions, logits, state, out_tokens, tok_in;
    DevBuf argmax_part, counters;  // step_end partials; step_end's completion counter (zero between launches)
    AttnPlan plan_decode{};
    bool fused = false;  // one token on the decode-row GEMVs (rowgemv.hip)
    bool decode_attn = false;  // one token's attention on k_attn_decode
    DevBuf attn_row;           // its output when it runs unsplit
    DevBuf rope_cs;            // the decode step's rotation table (cos, sin) per rotation index
    bool prefetch = false;     // attention's spare CUs read the next weights ahead (GCQ_DECODE_PREFETCH=1: on)
    DevBuf ytmp;         // a prompt chunk's mul_mat result in packed row order
    int pos = 0;
    // The captured decode step, one graph per bucket of kKvBucket KV lengths (step_graph).
    static constexpr int kKvBucket = 32;
    std::vector<hipGraphExec_t> execs;

    ~Llama() {
        for (hipGraphExec_t e : execs)
            if (e) (void) hipGraphExecDestroy(e);
        if (stream) (void) hipStreamDestroy(stream);
    }

    int add(const std::string & name, int type, int64_t rows, int64_t cols, bool random) {
        Tensor t;
        t.name = name;
        t.type = type;
        t.rows = rows;
        t.cols = cols;
        t.random = random;
        t.buf = DevBuf(type == T_F32 ? (size_t) rows * cols * 4 : weight_layout(type, rows, cols).total);
        tensors.push_back(std::move(t));
        return (int) tensors.size() - 1;
    }

    const Tensor & T(int i) const { return tensors[i]; }
    uint16_t * kv_layer(int l) const {
        return kv.as<uint16_t>() + (size_t) l * 2 * c.n_head_kv * c.max_ctx * c.head_dim;
    }

    void init(const gcq_llama_config & cfg, int max_prompt_) {
        c = cfg;
        max_prompt = max_prompt_;
        require(c.n_layer > 0 && c.n_embd > 0 && c.n_head > 0 && c.n_head_kv > 0 && c.head_dim > 0 && c.n_ff > 0 &&
                    c.n_vocab > 0 && c.max_ctx > 0,
                "llama: every size must be positive");
        require(c.n_vocab <= 524288, "llama: at most 524288 vocabulary entries (the greedy step's argmax)");
        require(c.wtype == T_Q4_0 || c.wtype == T_Q8_0, "llama: weight type must be Q4_0 or Q8_0");
        require(c.n_head % c.n_head_kv == 0 && c.n_head / c.n_head_kv <= 8, "llama: 1..8 query heads per KV head");
        require(c.head_dim == 64 || c.head_dim == 128, "llama: head_dim must be 64 or 128");
        require(c.n_embd % 256 == 0 && c.n_ff % 32 == 0 && ((int64_t) c.n_head * c.head_dim) % 32 == 0,
                "llama: n_embd must be a multiple of 256 and n_ff of 32");
        require(max_prompt >= 1 && max_prompt <= c.max_ctx, "llama: 1 <= max_prompt <= max_ctx");
        check_hip(hipStreamCreate(&stream), "hipStreamCreate");
        qkv_dim = (int64_t) (c.n_head + 2 * c.n_head_kv) * c.head_dim;
        attn_dim = (int64_t) c.n_head * c.head_dim;
        // Tensor order = seed order of init_random (tensor i draws from seed + i).
        t_embd = add("token_embd", c.wtype, c.n_vocab, c.n_embd, true);
        for (int l = 0; l < c.n_layer; l++) {
            const std::string b = "blk." + std::to_string(l) + ".";
            Layer L;
            L.attn_norm = add(b + "attn_norm", T_F32, 1, c.n_embd, false);
            L.qkv = add(b + "attn_qkv", c.wtype, qkv_dim, c.n_embd, true);
            L.wo = add(b + "attn_output", c.wtype, c.n_embd, attn_dim, true);
            L.ffn_norm = add(b + "ffn_norm", T_F32, 1, c.n_embd, false);
            L.gate_up = add(b + "ffn_gate_up", c.wtype, 2 * (int64_t) c.n_ff, c.n_embd, true);
            L.down = add(b + "ffn_down", c.wtype, c.n_embd, c.n_ff, true);
            layers.push_back(L);
        }
        t_out_norm = add("output_norm", T_F32, 1, c.n_embd, false);
        t_out = add("output", c.wtype, c.n_vocab, c.n_embd, true);

        const size_t kv_bytes = (size_t) c.n_layer * 2 * c.n_head_kv * c.max_ctx * c.head_dim * 2;
        kv = DevBuf(kv_bytes);
        x = DevBuf((size_t) max_prompt * c.n_embd * 4);
        qkv = DevBuf((size_t) max_prompt * qkv_dim * 4);
        gu = DevBuf((size_t) max_prompt * 2 * c.n_ff * 4);
        const int64_t widest = std::max<int64_t>({(int64_t) c.n_embd, (int64_t) c.n_ff, attn_dim});
        act_a = DevBuf(act_layout(c.wtype, max_prompt, widest).total);
        act_b = DevBuf(act_layout(c.wtype, max_prompt, widest).total);
        size_t po = 0, pml = 0;
        for (int S = 1; S <= max_prompt; S++) {
            const AttnPlan p = attn_plan(S, c.n_head_kv, c.max_ctx);
            po = std::max(po, (size_t) S * c.n_head * p.nsplit * c.head_dim * 4);
            pml = std::max(pml, (size_t) S * c.n_head * p.nsplit * 8);
        }
        // One token runs on the decode-row GEMVs when every projection's K fits them: QKV and
        // gate/up are then packed in row pairs (rope pairs, gate/up pairs) for their epilogues.
        decode_attn = attn_decode_fits(c.head_dim, c.n_head / c.n_head_kv);
        if (const char * e = std::getenv("GCQ_DECODE_PREFETCH")) prefetch = std::string(e) == "1";
        plan_decode = decode_attn ? attn_plan_decode(c.head_dim, c.n_head, c.n_head / c.n_head_kv, c.max_ctx,
                                                     row_gemv_merge_max())
                                  : attn_plan(1, c.n_head_kv, c.max_ctx);
        fused = row_gemv_fits(c.wtype, c.n_embd) && row_gemv_fits(c.wtype, attn_dim) &&
                row_gemv_fits(c.wtype, c.n_ff) && c.head_dim % 4 == 0 &&
                plan_decode.nsplit <= row_gemv_merge_max();
        attn_row = DevBuf((size_t) attn_dim * 4);
        rope_cs = DevBuf((size_t) c.head_dim / 2 * sizeof(float2));
        po = std::max(po, (size_t) c.n_head * plan_decode.nsplit * c.head_dim * 4);
        pml = std::max(pml, (size_t) c.n_head * plan_decode.nsplit * 8);
        if (fused) {
            const int D = c.head_dim, half = D / 2, nqk = (c.n_head + c.n_head_kv) * half;
            std::vector<int32_t> pq(qkv_dim), pg(2 * (size_t) c.n_ff);
            for (int64_t r = 0; r < qkv_dim; r++) {
                const int64_t g = r / 2, b = r % 2;
                pq[r] = (int32_t) (g < nqk ? (g / half) * D + g % half + b * half
                                           : (int64_t) (c.n_head + c.n_head_kv) * D + 2 * (g - nqk) + b);
            }
            for (int64_t r = 0; r < 2 * (int64_t) c.n_ff; r++) pg[r] = (int32_t) ((r % 2) * c.n_ff + r / 2);
            for (const Layer & L : layers) {
                set_perm(L.qkv, pq);
                set_perm(L.gate_up, pg);
            }
            ytmp = DevBuf((size_t) max_prompt * std::max<int64_t>(qkv_dim, 2 * (int64_t) c.n_ff) * 4);
        }
        part_o = DevBuf(po);
        part_ml = DevBuf(pml);
        mask = DevBuf((size_t) max_prompt * c.max_ctx * 2);
        positions = DevBuf((size_t) max_prompt * 4);
        tok_in = DevBuf((size_t) max_prompt * 4);
        logits = DevBuf((size_t) c.n_vocab * 4);
        state = DevBuf(sizeof(StepStateHost));
        out_tokens = DevBuf((size_t) c.max_ctx * 4);
        argmax_part = DevBuf(256 * sizeof(float2));
        counters = DevBuf(4096);
        check_hip(hipMemset(counters.p, 0, counters.n), "counters");
        std::vector<float> ones(c.n_embd, 1.0f);
        for (auto & t : tensors)
            if (t.type == T_F32)
                check_hip(hipMemcpy(t.buf.p, ones.data(), (size_t) t.cols * 4, hipMemcpyHostToDevice), "norm init");
        reset();
    }

    void set_perm(int ti, const std::vector<int32_t> & map) {
        Tensor & t = tensors[ti];
        t.perm = DevBuf(map.size() * 4);
        check_hip(hipMemcpy(t.perm.p, map.data(), map.size() * 4, hipMemcpyHostToDevice), "perm");
    }

    // ggml block rows on the device (raw, natural order) -> the tensor's packed buffer.
    void pack_into(Tensor & t, const void * raw, void * tmp) {
        const void * src = raw;
        if (t.perm.p) {
            launch_move_rows(raw, tmp, t.perm.as<int32_t>(), t.rows, row_bytes(t.type, t.cols), false, stream);
            src = tmp;
        }
        launch_pack(t.type, src, t.rows, t.cols, t.buf.p, stream);
    }

    void reset() {
        check_hip(hipMemsetAsync(kv.p, 0, kv.n, stream), "KV reset");
        check_hip(hipStreamSynchronize(stream), "sync");
        pos = 0;
    }

    // Weights: N(0, stddev^2) from the counter-based stream (tensor i: seed + i), encoded on the GPU.
    void init_random(uint64_t seed, float stddev) {
        size_t biggest = 0;
        for (auto & t : tensors)
            if (t.random) biggest = std::max(biggest, (size_t) (t.rows * t.cols));
        DevBuf f32(biggest * 4), raw(biggest / 32 * 34 + 256), tmp(biggest / 32 * 34 + 256);
        for (size_t i = 0; i < tensors.size(); i++) {
            Tensor & t = tensors[i];
            if (!t.random) continue;
            launch_fill_normal(f32.as<float>(), t.rows * t.cols, seed + i, 0, stddev, stream);
            launch_encode(t.type, f32.as<float>(), t.rows, t.cols, raw.p, stream);
            pack_into(t, raw.p, tmp.p);
        }
        check_hip(hipStreamSynchronize(stream), "init_random");
    }

    int find(const char * name) const {
        require(name != nullptr, "weight name is NULL");
        for (size_t i = 0; i < tensors.size(); i++)
            if (tensors[i].name == name) return (int) i;
        fail(std::string("no weight named '") + name + "'");
    }

    void set_weight(const char * name, const void * host, size_t nbytes) {
        Tensor & t = tensors[find(name)];
        const size_t want = t.type == T_F32 ? (size_t) t.cols * 4 : row_bytes(t.type, t.cols) * t.rows;
        require(nbytes == want, std::string(name) + ": " + std::to_string(nbytes) + " bytes given, " +
                                    std::to_string(want) + " expected (ggml block bytes)");
        require(host != nullptr, "data is NULL");
        if (t.type == T_F32) {
            check_hip(hipMemcpy(t.buf.p, host, nbytes, hipMemcpyHostToDevice), "set_weight");
            return;
        }
        DevBuf raw(nbytes), tmp(t.perm.p ? nbytes : 0);
        check_hip(hipMemcpy(raw.p, host, nbytes, hipMemcpyHostToDevice), "set_weight");
        pack_into(t, raw.p, tmp.p);
        check_hip(hipStreamSynchronize(stream), "set_weight");
    }

    void get_weight(const char * name, void * host, size_t nbytes) const {
        const Tensor & t = tensors[find(name)];
        const size_t want = t.type == T_F32 ? (size_t) t.cols * 4 : row_bytes(t.type, t.cols) * t.rows;
        require(nbytes == want, std::string(name) + ": buffer of " + std::to_string(nbytes) + " bytes, need " +
                                    std::to_string(want));
        require(host != nullptr, "data is NULL");
        if (t.type == T_F32) {
            check_hip(hipMemcpy(host, t.buf.p, nbytes, hipMemcpyDeviceToHost), "get_weight");
            return;
        }
        DevBuf raw(nbytes), tmp(t.perm.p ? nbytes : 0);
        launch_unpack(t.type, t.buf.p, t.rows, t.cols, raw.p, stream);
        if (t.perm.p) launch_move_rows(raw.p, tmp.p, t.perm.as<int32_t>(), t.rows, nbytes / t.rows, true, stream);
        check_hip(hipStreamSynchronize(stream), "get_weight");
        check_hip(hipMemcpy(host, (t.perm.p ? tmp : raw).p, nbytes, hipMemcpyDeviceToHost), "get_weight");
    }

    void mul_mat(int ti, const void * act, int64_t S, float * y, int64_t ldy, const float * res) {
        const Tensor & t = tensors[ti];
        float * out = y;
        int64_t ldo = ldy;
        if (t.perm.p) {  // rows packed in pairs: compute in packed order, then put columns back
            require(res == nullptr, "mul_mat: residual on a row-paired weight");
            out = ytmp.as<float>();
            ldo = t.rows;
        }
        if (S <= 8) launch_gemv(t.type, t.buf.p, t.rows, t.cols, act, S, out, ldo, stream, res);
        else launch_gemm(t.type, t.buf.p, t.rows, t.cols, act, S, out, ldo, stream, res);
        if (t.perm.p) launch_scatter_cols(out, ldo, y, ldy, t.perm.as<int32_t>(), (int) S, (int) t.rows, stream);
    }

    RowArgs row_args(int ti) const {
        const Tensor & t = tensors[ti];
        const WeightLayout W = weight_layout(t.type, t.rows, t.cols);
        RowArgs a{};
        a.wqs = t.buf.as<uint8_t>() + W.qs;
        a.wd = reinterpret_cast<const uint16_t *>(t.buf.as<uint8_t>() + W.d);
        a.N = (int) t.rows;
        a.nb = (int) (t.cols / QK);
        return a;
    }

    // The single-token forward on the decode-row GEMVs: per layer QKV (rms_norm in, rope + K/V
    // cache out), split-K attention, output projection (merge in, residual out), gate/up
    // (rms_norm in, swiglu out), down (residual out); then the lm head (rms_norm in).
    void forward_one(const int32_t * tok_dev, const int32_t * pos_dev, int n_kv, const int * n_kv_dev,
                     const AttnPlan & plan) {
        float * xs = x.as<float>();
        const Tensor & E = tensors[t_embd];
        launch_embed_rope(E.type, E.buf.p, E.rows, E.cols, tok_dev, xs, pos_dev, c.head_dim, c.rope_base, rope_cs.p,
                          stream);
        for (int l = 0; l < c.n_layer; l++) decode_layer(l, pos_dev, n_kv, n_kv_dev, plan, nullptr);
        RowArgs a = row_args(t_out);
        a.x = xs;
        a.norm_w = tensors[t_out_norm].buf.as<float>();
        a.eps = c.rms_eps;
        a.y = logits.as<float>();
        launch_row_gemv(c.wtype, PRO_NORM, EPI_STORE, a, stream);
    }

    // Layer l of the single-token forward on the residual row x (the rotation table of the
    // position already in rope_cs). n_kv: the most keys the step may see (the KV length itself is
    // read from n_kv_dev); the attention's splits cover cache rows [0, n_kv) only. mid (device,
    // optional): the residual after attention.
    void decode_layer(int l, const int32_t * pos_dev, int n_kv, const int * n_kv_dev, const AttnPlan & plan,
                      float * mid) {
        float * xs = x.as<float>();
        const float scale = 1.0f / std::sqrt((float) c.head_dim);
        const int64_t kv_h = (int64_t) c.max_ctx * c.head_dim;
        const Layer & L = layers[l];
        uint16_t * kvl = kv_layer(l);
        RowArgs a = row_args(L.qkv);
        a.x = xs;
        a.norm_w = tensors[L.attn_norm].buf.as<float>();
        a.eps = c.rms_eps;
        a.y = qkv.as<float>();
        a.pos = pos_dev;
        a.kc = kvl;
        a.vc = kvl + (size_t) c.n_head_kv * kv_h;
        a.ctx = c.max_ctx;
        a.H = c.n_head;
        a.Hkv = c.n_head_kv;
        a.D = c.head_dim;
        a.rope_cs = rope_cs.as<float2>();
        launch_row_gemv(c.wtype, PRO_NORM, EPI_ROPE_KV, a, stream);
        if (decode_attn) {
            // Spare CUs read this layer's output projection and the next layer's QKV weights
            // into the Infinity Cache while the attention runs.
            Prefetch pf;
            pf.p[0] = tensors[L.wo].buf.as<uint8_t>();
            pf.n[0] = tensors[L.wo].buf.n & ~(size_t) 15;
            if (l + 1 < c.n_layer) {
                pf.p[1] = tensors[layers[l + 1].qkv].buf.as<uint8_t>();
                pf.n[1] = tensors[layers[l + 1].qkv].buf.n & ~(size_t) 15;
            }
            pf.sink = counters.as<unsigned int>() + 64;
            launch_attn_decode(qkv.as<float>(), c.head_dim, kvl, kv_h, c.head_dim, kvl + (size_t) c.n_head_kv * kv_h,
                               kv_h, c.head_dim, c.head_dim, c.n_head, c.n_head_kv, n_kv, n_kv_dev, scale,
                               plan.nsplit, plan.chunk, n_kv, decode_group(c.n_head / c.n_head_kv, n_kv),
                               attn_row.as<float>(), part_o.as<float>(), part_ml.as<float2>(), stream,
                               prefetch ? &pf : nullptr, nullptr, 16);
        } else {
            launch_attn_split(qkv.as<float>(), c.head_dim, qkv_dim, kvl, kv_h, c.head_dim,
                              kvl + (size_t) c.n_head_kv * kv_h, kv_h, c.head_dim, nullptr, n_kv, c.head_dim, 1,
                              c.n_head, c.n_head_kv, n_kv, scale, part_o.as<float>(), part_ml.as<float2>(), plan,
                              n_kv_dev, stream);
        }
        a = row_args(L.wo);
        a.y = xs;
        a.res = xs;
        if (decode_attn && plan.nsplit == 1) {  // the attention row itself
            a.x = attn_row.as<float>();
            launch_row_gemv(c.wtype, PRO_PLAIN, EPI_STORE, a, stream);
        } else {  // its split-K partials, merged in the prologue
            a.part_o = part_o.as<float>();
            a.part_ml = part_ml.as<float2>();
            a.nsplit = plan.nsplit;
            a.D = c.head_dim;
            launch_row_gemv(c.wtype, PRO_MERGE, EPI_STORE, a, stream);
        }
        if (mid) check_hip(hipMemcpyAsync(mid, xs, (size_t) c.n_embd * 4, hipMemcpyDeviceToDevice, stream), "mid");
        ffn_decode(L, xs);
    }

    // The feed-forward half of a decode layer on the residual row xs: rms_norm -> gate/up ->
    // SwiGLU in one launch, then down + residual.
    void ffn_decode(const Layer & L, float * xs) {
        RowArgs a = row_args(L.gate_up);
        a.x = xs;
        a.norm_w = tensors[L.ffn_norm].buf.as<float>();
        a.eps = c.rms_eps;
        a.y = gu.as<float>();
        launch_row_gemv(c.wtype, PRO_NORM, EPI_SWIGLU, a, stream);
        a = row_args(L.down);
        a.x = gu.as<float>();
        a.y = xs;
        a.res = xs;
        launch_row_gemv(c.wtype, PRO_PLAIN, EPI_STORE, a, stream);
    }

    // ggml_rms_norm + ggml_mul by norm t_norm of S rows of the residual stream (the last row only
    // when last_only), then mul_mat by weight ti into y. One row: a single launch, the GEMV
    // quantizing the normalized row itself where the shape allows; else rmsnorm_q8 into act_a first.
    void norm_mul_mat(int t_norm, int ti, const float * xs, int S, bool last_only, float * y, int64_t ldy) {
        const Tensor & t = tensors[ti];
        const float * nw = tensors[t_norm].buf.as<float>();
        const int rows = last_only ? 1 : S;
        const float * xr = xs + (size_t) (S - rows) * c.n_embd;
        if (rows == 1 && !t.perm.p && row_gemv_fits(t.type, t.cols)) {
            RowArgs a = row_args(ti);
            a.x = xr;
            a.norm_w = nw;
            a.eps = c.rms_eps;
            a.y = y;
            return launch_row_gemv(t.type, PRO_NORM, EPI_STORE, a, stream);
        }
        launch_rmsnorm_q8(xr, c.n_embd, nw, c.rms_eps, rows, c.n_embd, act_a.p, stream);
        mul_mat(ti, act_a.p, rows, y, ldy, nullptr);
    }

    // S tokens at positions pos_dev[0..S) (device), the last of which sees n_kv keys. Decode (the
    // captured step) passes the state's position / KV length pointers and no mask.
    void forward(int S, const int32_t * tok_dev, const int32_t * pos_dev, int n_kv, const int * n_kv_dev,
                 const void * mask_dev, const AttnPlan & plan) {
        if (S == 1 && fused && mask_dev == nullptr) return forward_one(tok_dev, pos_dev, n_kv, n_kv_dev, plan);
        float * xs = x.as<float>();
        const Tensor & E = tensors[t_embd];
        launch_get_rows(E.type, E.buf.p, E.rows, E.cols, tok_dev, S, xs, stream);
        for (int l = 0; l < c.n_layer; l++) prompt_layer(l, S, pos_dev, n_kv, n_kv_dev, mask_dev, plan, nullptr);
        norm_mul_mat(t_out_norm, t_out, xs, S, true, logits.as<float>(), c.n_vocab);
    }

    // Layer l of a prompt chunk of S rows of the residual stream x. mid (device, optional): the
    // rows after attention.
    void prompt_layer(int l, int S, const int32_t * pos_dev, int n_kv, const int * n_kv_dev, const void * mask_dev,
                      const AttnPlan & plan, float * mid) {
        float * xs = x.as<float>();
        const float scale = 1.0f / std::sqrt((float) c.head_dim);
        const int64_t kv_h = (int64_t) c.max_ctx * c.head_dim;
        const Layer & L = layers[l];
        uint16_t * kvl = kv_layer(l);
        norm_mul_mat(L.attn_norm, L.qkv, xs, S, false, qkv.as<float>(), qkv_dim);
        launch_rope_kv(qkv.as<float>(), qkv_dim, pos_dev, S, c.n_head, c.n_head_kv, c.head_dim, c.rope_base, kvl,
                       c.max_ctx, stream);
        launch_attn_split(qkv.as<float>(), c.head_dim, qkv_dim, kvl, kv_h, c.head_dim, kvl + (size_t) c.n_head_kv * kv_h,
                          kv_h, c.head_dim, mask_dev, n_kv, c.head_dim, S, c.n_head, c.n_head_kv, n_kv, scale,
                          part_o.as<float>(), part_ml.as<float2>(), plan, n_kv_dev, stream);
        launch_merge_q8(part_o.as<float>(), part_ml.as<float2>(), plan.nsplit, S, c.n_head, c.head_dim, nullptr,
                        act_b.p, stream);
        mul_mat(L.wo, act_b.p, S, xs, c.n_embd, xs);
        if (mid) check_hip(hipMemcpyAsync(mid, xs, (size_t) S * c.n_embd * 4, hipMemcpyDeviceToDevice, stream), "mid");
        norm_mul_mat(L.ffn_norm, L.gate_up, xs, S, false, gu.as<float>(), 2 * (int64_t) c.n_ff);
        launch_swiglu_q8(gu.as<float>(), gu.as<float>() + c.n_ff, 2 * (int64_t) c.n_ff, c.n_ff, S, act_b.p, stream);
        mul_mat(L.down, act_b.p, S, xs, c.n_embd, xs);
    }

    // Layers [first, first + count) on n given residual rows (host, n x n_embd) at positions
    // pos0 .. pos0 + n - 1, with the kernels a prompt chunk (n > 1) or the decode step (n == 1)
    // runs, their K / V written into the cache at those positions. x_out (host, n x n_embd): the
    // last layer's output; mid (host, count x n x n_embd, optional): each layer's rows after
    // attention. The model's position is left as it is.
    void forward_layers(const float * x_in, int n, int pos0, int first, int count, float * x_out, float * mid) {
        require(n >= 1 && n <= max_prompt, "forward_layers: 1 <= n <= max_prompt");
        require(pos0 >= 0 && pos0 + n <= c.max_ctx, "forward_layers: positions past max_ctx");
        require(first >= 0 && count >= 1 && first + count <= c.n_layer, "forward_layers: layer range out of range");
        const size_t row_bytes = (size_t) n * c.n_embd * 4;
        DevBuf mid_dev(mid ? row_bytes * count : 0);
        float * xs = x.as<float>();
        if (n == 1 && fused) {
            // the decode step's state: position, KV length and a token whose embedding row and the
            // position's rotation table the step's first launch makes (the row is replaced below)
            const StepStateHost st{pos0, pos0 + 1, 0, 0};
            check_hip(hipMemcpyAsync(state.p, &st, sizeof st, hipMemcpyHostToDevice, stream), "state");
            StepStateHost * sd = state.as<StepStateHost>();
            const Tensor & E = tensors[t_embd];
            launch_embed_rope(E.type, E.buf.p, E.rows, E.cols, &sd->token, xs, &sd->pos, c.head_dim, c.rope_base,
                              rope_cs.p, stream);
            check_hip(hipMemcpyAsync(xs, x_in, row_bytes, hipMemcpyHostToDevice, stream), "x");
            for (int l = first; l < first + count; l++)
                decode_layer(l, &sd->pos, c.max_ctx, &sd->n_kv, plan_decode,
                             mid ? mid_dev.as<float>() + (size_t) (l - first) * n * c.n_embd : nullptr);
        } else {
            std::vector<int32_t> p(n);
            for (int j = 0; j < n; j++) p[j] = pos0 + j;
            check_hip(hipMemcpyAsync(positions.p, p.data(), n * 4, hipMemcpyHostToDevice, stream), "positions");
            check_hip(hipMemcpyAsync(xs, x_in, row_bytes, hipMemcpyHostToDevice, stream), "x");
            const int n_kv = pos0 + n;
            launch_causal_mask(mask.p, n, n_kv, pos0, stream);
            const AttnPlan plan = attn_plan(n, c.n_head_kv, n_kv);
            for (int l = first; l < first + count; l++)
                prompt_layer(l, n, positions.as<int32_t>(), n_kv, nullptr, mask.p, plan,
                             mid ? mid_dev.as<float>() + (size_t) (l - first) * n * c.n_embd : nullptr);
        }
        check_hip(hipStreamSynchronize(stream), "forward_layers");
        check_hip(hipMemcpy(x_out, xs, row_bytes, hipMemcpyDeviceToHost), "x_out");
        if (mid) check_hip(hipMemcpy(mid, mid_dev.p, row_bytes * count, hipMemcpyDeviceToHost), "mid");
    }

    void prefill(const int32_t * tokens, int n, float * logits_host) {
        require(n >= 1, "prefill: at least one token");
        require(pos + n <= c.max_ctx, "context full: " + std::to_string(pos) + " + " + std::to_string(n) +
                                          " tokens > max_ctx " + std::to_string(c.max_ctx));
        for (int i = 0; i < n; i += max_prompt) {
            const int S = std::min(max_prompt, n - i);
            std::vector<int32_t> p(S);
            for (int j = 0; j < S; j++) p[j] = pos + j;
            check_hip(hipMemcpyAsync(positions.p, p.data(), S * 4, hipMemcpyHostToDevice, stream), "positions");
            check_hip(hipMemcpyAsync(tok_in.p, tokens + i, S * 4, hipMemcpyHostToDevice, stream), "tokens");
            const int n_kv = pos + S;
            launch_causal_mask(mask.p, S, n_kv, pos, stream);
            forward(S, tok_in.as<int32_t>(), positions.as<int32_t>(), n_kv, nullptr, mask.p,
                    attn_plan(S, c.n_head_kv, n_kv));
            check_hip(hipStreamSynchronize(stream), "prefill");
            pos += S;
        }
        if (logits_host)
            check_hip(hipMemcpy(logits_host, logits.p, (size_t) c.n_vocab * 4, hipMemcpyDeviceToHost), "logits");
    }

    // The attention plan of a decode step that sees at most n_kv keys.
    AttnPlan decode_plan(int n_kv) const {
        return decode_attn ? attn_plan_decode(c.head_dim, c.n_head, c.n_head / c.n_head_kv, n_kv, row_gemv_merge_max())
                           : attn_plan(1, c.n_head_kv, n_kv);
    }

    // The captured decode step for a step that sees n_kv keys: one graph per bucket of kKvBucket
    // KV lengths, its attention planned and its K / V rows read for the bucket's largest length
    // (so the step's work follows the position, not max_ctx), instantiated on first use. Token,
    // position and KV length come from the device state; step_end advances it.
    hipGraphExec_t step_graph(int n_kv) {
        require(n_kv >= 1 && n_kv <= c.max_ctx, "decode: KV length out of range");
        const size_t b = (size_t) (n_kv - 1) / kKvBucket;
        if (execs.size() <= b) execs.resize(b + 1, nullptr);
        if (execs[b]) return execs[b];
        const int bound = std::min(c.max_ctx, (int) (b + 1) * kKvBucket);
        (void) cu_count();  // device queries happen before capture
        StepStateHost * st = state.as<StepStateHost>();
        hipGraph_t g = nullptr;
        check_hip(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "capture");
        try {
            forward(1, &st->token, &st->pos, bound, &st->n_kv, nullptr, decode_plan(bound));
            launch_step_end(logits.as<float>(), c.n_vocab, state.p, out_tokens.as<int32_t>(), c.max_ctx,
                            argmax_part.p, counters.as<unsigned int>() + 0, stream);
        } catch (...) {
            (void) hipStreamEndCapture(stream, &g);
            if (g) (void) hipGraphDestroy(g);
            throw;
        }
        check_hip(hipStreamEndCapture(stream, &g), "capture end");
        const hipError_t e = hipGraphInstantiate(&execs[b], g, nullptr, nullptr, 0);
        (void) hipGraphDestroy(g);
        check_hip(e, "graph instantiate");
        return execs[b];
    }

    // Instantiates the step graphs a decode up to KV length n_kv may launch, before any of them is
    // launched: every bucket up to max_ctx on the first call when there are at most 128 (a few
    // tenths of a ms each), else the buckets up to n_kv.
    void prepare_graphs(int n_kv) {
        const int buckets = (c.max_ctx + kKvBucket - 1) / kKvBucket;
        const int upto = buckets <= 128 ? c.max_ctx : n_kv;
        for (int b = 0; b * kKvBucket < upto; b++) (void) step_graph(std::min(upto, (b + 1) * kKvBucket));
    }

    void set_state(int token) {
        const StepStateHost st{pos, pos + 1, token, 0};
        check_hip(hipMemcpyAsync(state.p, &st, sizeof st, hipMemcpyHostToDevice, stream), "state");
    }

    void decode(int32_t token, float * logits_host, int32_t * next) {
        require(token >= 0 && token < c.n_vocab, "token id out of range");
        require(pos + 1 <= c.max_ctx, "context full");
        prepare_graphs(pos + 1);
        hipGraphExec_t step = step_graph(pos + 1);
        set_state(token);
        check_hip(hipGraphLaunch(step, stream), "graph launch");
        check_hip(hipStreamSynchronize(stream), "decode");
        pos += 1;
        if (logits_host)
            check_hip(hipMemcpy(logits_host, logits.p, (size_t) c.n_vocab * 4, hipMemcpyDeviceToHost), "logits");
        if (next) {
            StepStateHost st;
            check_hip(hipMemcpy(&st, state.p, sizeof st, hipMemcpyDeviceToHost), "state");
            *next = st.token;
        }
    }

    void generate(int32_t first, int n_new, int32_t * out) {
        require(first >= 0 && first < c.n_vocab, "token id out of range");
        require(n_new >= 0 && pos + n_new <= c.max_ctx, "context full: generate would pass max_ctx");
        if (n_new == 0) return;
        prepare_graphs(pos + n_new);
        set_state(first);
        for (int i = 0; i < n_new; i++) check_hip(hipGraphLaunch(step_graph(pos + i + 1), stream), "graph launch");
        check_hip(hipStreamSynchronize(stream), "generate");
        pos += n_new;
        if (out) check_hip(hipMemcpy(out, out_tokens.p, (size_t) n_new * 4, hipMemcpyDeviceToHost), "tokens");
    }
};

}  // namespace gcq

using namespace gcq;

struct gcq_llama : Llama {};

extern "C" {

gcq_llama * gcq_llama_create(const gcq_llama_config * cfg, int max_prompt) {
    gcq_llama * m = nullptr;
    const int rc = guarded([&] {
        require(cfg != nullptr, "config is NULL");
        require(gcq_device_count() > 0, "no HIP device");
        std::unique_ptr<gcq_llama> p(new gcq_llama());
        p->init(*cfg, max_prompt);
        m = p.release();
    });
    return rc == 0 ? m : nullptr;
}

void gcq_llama_free(gcq_llama * m) { delete m; }

int gcq_llama_init_random(gcq_llama * m, uint64_t seed, float stddev) {
    return guarded([&] {
        require(m != nullptr, "model is NULL");
        m->init_random(seed, stddev);
    });
}

int gcq_llama_n_weights(const gcq_llama * m) { return m ? (int) m->tensors.size() : -1; }

int gcq_llama_weight_info(const gcq_llama * m, int i, const char ** name, int * type, int64_t * rows, int64_t * cols) {
    return guarded([&] {
        require(m != nullptr, "model is NULL");
        require(i >= 0 && i < (int) m->tensors.size(), "weight index out of range");
        const auto & t = m->tensors[i];
        if (name) *name = t.name.c_str();
        if (type) *type = t.type;
        if (rows) *rows = t.rows;
        if (cols) *cols = t.cols;
    });
}

int gcq_llama_set_weight(gcq_llama * m, const char * name, const void * data, size_t nbytes) {
    return guarded([&] {
        require(m != nullptr, "model is NULL");
        m->set_weight(name, data, nbytes);
    });
}

int gcq_llama_get_weight(const gcq_llama * m, const char * name, void * data, size_t nbytes) {
    return guarded([&] {
        require(m != nullptr, "model is NULL");
        m->get_weight(name, data, nbytes);
    });
}

int gcq_llama_reset(gcq_llama * m) {
    return guarded([&] {
        require(m != nullptr, "model is NULL");
        m->reset();
    });
}

int gcq_llama_position(const gcq_llama * m) { return m ? m->pos : -1; }

int gcq_llama_prefill(gcq_llama * m, const int32_t * tokens, int n, float * logits) {
    return guarded([&] {
        require(m != nullptr && tokens != nullptr, "model or tokens is NULL");
        for (int i = 0; i < n; i++) require(tokens[i] >= 0 && tokens[i] < m->c.n_vocab, "token id out of range");
        m->prefill(tokens, n, logits);
    });
}

int gcq_llama_decode(gcq_llama * m, int32_t token, float * logits, int32_t * next) {
    return guarded([&] {
        require(m != nullptr, "model is NULL");
        m->decode(token, logits, next);
    });
}

int gcq_llama_forward_layers(gcq_llama * m, const float * x, int n, int pos, int first_layer, int n_layers, float * x_out,
                             float * x_mid) {
    return guarded([&] {
        require(m != nullptr && x != nullptr && x_out != nullptr, "model, x or x_out is NULL");
        m->forward_layers(x, n, pos, first_layer, n_layers, x_out, x_mid);
    });
}

int gcq_llama_generate(gcq_llama * m, int32_t first, int n_new, int32_t * out_tokens) {
    return guarded([&] {
        require(m != nullptr, "model is NULL");
        m->generate(first, n_new, out_tokens);
    });
}

}  // extern "C"
