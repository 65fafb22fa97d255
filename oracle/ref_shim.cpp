// ref_shim.cpp — TEST INFRASTRUCTURE ONLY.  Exposes the reference's own CPU QK-norm and
// RoPE functions, compiled from the reference sources where they lie (-I <reference>/src),
// behind extern "C" entry points so the oracle restatement can be compared bit for bit.
//
//   elref_rmsnorm        -> el::rmsnorm        (src/ops.cpp:155-160)
//   elref_rope_inv_freq  -> el::rope_inv_freq  (src/model.cpp:105-109)
//   elref_rope           -> el::rope           (src/model.cpp:23-32; file-local, hence the
//                                                include of model.cpp into this unit)
//
// Everything else in those files (CpuModel, read_config, the GGUF tensor table) is left
// unreferenced and dropped by --gc-sections: it needs src/gguf.cpp, which includes
// <windows.h> and does not build here.
#include "model.cpp"
#include "ops.h"

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
