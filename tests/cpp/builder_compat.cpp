// A stage builder written the way ggml-compiler's C++ emitter writes them (ggml calls, and the
// multi-call helpers of runtime/include/ggml_compiler_ops.h: mul_mat with f32 accumulation,
// flash_attn with a backend support query, slice, reshape, scale), compiled against libgcq's
// ggml.h: one decoder layer's decode step. Builds the graph on the host only and prints its
// node ops, one per line, then "nodes N".
#include <cmath>
#include <cstdio>

#include "ggml-backend.h"
#include "ggml.h"
#include "ggml_compiler_ops.h"

int main() {
    const int64_t E = 256, H = 4, Hkv = 2, D = 64, F = 512, CTX = 256, NKV = 256;
    ggml_init_params ip = {1 << 20, nullptr, true};
    ggml_context * ctx = ggml_init(ip);
    ggml_tensor * x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, E, 1);
    ggml_tensor * pos = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, 1);
    ggml_tensor * mask = ggml_new_tensor_2d(ctx, GGML_TYPE_F16, NKV, 1);
    ggml_tensor * attn_norm = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, E);
    ggml_tensor * wq = ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_0, E, H * D);
    ggml_tensor * wk = ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_0, E, Hkv * D);
    ggml_tensor * wv = ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_0, E, Hkv * D);
    ggml_tensor * wo = ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_0, H * D, E);
    ggml_tensor * ffn_norm = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, E);
    ggml_tensor * wg = ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_0, E, F);
    ggml_tensor * wu = ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_0, E, F);
    ggml_tensor * wd = ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_0, F, E);
    ggml_tensor * kc = ggml_new_tensor_3d(ctx, GGML_TYPE_F16, D, CTX, Hkv);
    ggml_tensor * vc = ggml_new_tensor_3d(ctx, GGML_TYPE_F16, D, CTX, Hkv);
    auto supported = [](ggml_tensor * t) { return t->ne[0] == 64 || t->ne[0] == 128; };

    ggml_tensor * t0 = ggml_rms_norm(ctx, x, 1e-05f);
    ggml_tensor * t1 = ggml_mul(ctx, t0, attn_norm);
    ggml_tensor * t2 = ggml_compiler::ops::mul_mat(ctx, wq, t1, true);
    ggml_tensor * t3 = ggml_compiler::ops::mul_mat(ctx, wk, t1, true);
    ggml_tensor * t4 = ggml_compiler::ops::mul_mat(ctx, wv, t1, true);
    ggml_tensor * t5 = ggml_compiler::ops::reshape(ctx, t2, D, H, 1, 1);
    ggml_tensor * t6 = ggml_compiler::ops::reshape(ctx, t3, D, Hkv, 1, 1);
    ggml_tensor * t7 = ggml_compiler::ops::reshape(ctx, t4, D, Hkv, 1, 1);
    ggml_tensor * t8 = ggml_rope_ext(ctx, t5, pos, nullptr, 64, 2, 0, 10000.0f, 1.0f, 0.0f, 1.0f, 32.0f, 1.0f);
    ggml_tensor * t9 = ggml_rope_ext(ctx, t6, pos, nullptr, 64, 2, 0, 10000.0f, 1.0f, 0.0f, 1.0f, 32.0f, 1.0f);
    ggml_tensor * t10 = ggml_set_rows(ctx, kc, ggml_permute(ctx, t9, 0, 2, 1, 3), pos);
    ggml_tensor * t11 = ggml_set_rows(ctx, vc, ggml_permute(ctx, t7, 0, 2, 1, 3), pos);
    ggml_tensor * t12 = ggml_compiler::ops::slice(ctx, t10, 1, 0, D, NKV, Hkv, 1);
    ggml_tensor * t13 = ggml_compiler::ops::slice(ctx, t11, 1, 0, D, NKV, Hkv, 1);
    ggml_tensor * t14 = ggml_compiler::ops::flash_attn(ctx, ggml_permute(ctx, t8, 0, 2, 1, 3), t12, t13, mask,
                                                       0.125f, supported);
    ggml_tensor * t15 = ggml_compiler::ops::reshape(ctx, t14, D * H, 1, 1, 1);
    ggml_tensor * t16 = ggml_add(ctx, x, ggml_compiler::ops::mul_mat(ctx, wo, t15, true));
    ggml_tensor * t17 = ggml_mul(ctx, ggml_rms_norm(ctx, t16, 1e-05f), ffn_norm);
    ggml_tensor * t18 = ggml_swiglu_split(ctx, ggml_compiler::ops::mul_mat(ctx, wg, t17, true),
                                          ggml_compiler::ops::mul_mat(ctx, wu, t17, true));
    ggml_tensor * t19 = ggml_add(ctx, t16, ggml_compiler::ops::scale(ctx, ggml_compiler::ops::mul_mat(ctx, wd, t18, true),
                                                                      1.0f, 0.0f));
    if (!t19) {
        std::printf("error %s\n", ggml_last_error());
        return 1;
    }
    ggml_cgraph * g = ggml_new_graph(ctx);
    ggml_build_forward_expand(g, t19);
    for (int i = 0; i < ggml_graph_n_nodes(g); i++) std::printf("%s\n", ggml_op_desc(ggml_graph_node(g, i)));
    std::printf("nodes %d\n", ggml_graph_n_nodes(g));
    ggml_free(ctx);
    return 0;
}
