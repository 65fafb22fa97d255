// ref_shim.cpp — TEST INFRASTRUCTURE ONLY.  Exposes the reference's own CPU QK-norm and
// RoPE functions, compiled from the reference sources where they lie (-I <reference>/src),
// behind extern "C" entry points so the oracle restatement can be compared bit for bit.
//
//   elref_rmsnorm        -> el::rmsnorm        (src/ops.cpp:155-160)
//   elref_rope_inv_freq  -> el::rope_inv_freq  (src/model.cpp:105-109)
//   elref_rope           -> el::rope           (src/model.cpp:23-32; file-local, hence the
//                                                include of model.cpp into this unit)
//   elref_f16_to_f32     -> el::f16_to_f32     (src/ops.cpp:22-24)
//   elref_dot_f32        -> dot_f32            (src/ops.cpp:108-118; file-local, hence the
//   elref_dot_f16        -> dot_f16             include of ops.cpp into this unit, :92-106)
//   elref_dequant_q8_0   -> el::dequant_q8_0   (src/quant.cpp:7-13)
//   elref_dequant_q4_K   -> el::dequant_q4_K   (src/quant.cpp:15-33)
//   elref_dequant_q6_K   -> el::dequant_q6_K   (src/quant.cpp:35-60)
//
// Everything else in those files (CpuModel, read_config, the GGUF tensor table) is left
// unreferenced and dropped by --gc-sections: it needs src/gguf.cpp, which includes
// <windows.h> and does not build here.
#include "model.cpp"
#include "ops.cpp"
#include "ops.h"
#include "quant.h"

#define REF_API extern "C" __attribute__((visibility("default")))

REF_API void elref_rmsnorm(float* out, const float* x, const float* w, int n, float eps) {
    el::rmsnorm(out, x, w, n, eps);
}

REF_API void elref_rope_inv_freq(double* out, int rope_dim, double base) {
    el::Config c;
    c.rope_dim = rope_dim;
    c.rope_base = base;
    const std::vector<double> f = el::rope_inv_freq(c);
    for (size_t i = 0; i < f.size(); ++i) out[i] = f[i];
}

REF_API void elref_rope(float* v, int pos, int dim, const double* inv_freq) {
    const std::vector<double> f(inv_freq, inv_freq + dim / 2);
    el::rope(v, pos, dim, f);
}

REF_API float elref_f16_to_f32(uint16_t h) { return el::f16_to_f32(h); }

REF_API float elref_dot_f32(const float* w, const float* x, long n) { return el::dot_f32(w, x, n); }

REF_API float elref_dot_f16(const uint16_t* w, const float* x, long n) { return el::dot_f16(w, x, n); }

REF_API void elref_dequant_q8_0(const void* src, float* y, long n) { el::dequant_q8_0(src, y, n); }

REF_API void elref_dequant_q4_K(const void* src, float* y, long n) { el::dequant_q4_K(src, y, n); }

REF_API void elref_dequant_q6_K(const void* src, float* y, long n) { el::dequant_q6_K(src, y, n); }
