"""A tiny random-weight Qwen3 forward pass in numpy: the end-to-end harness for the attention path.

Test infrastructure only.  No Qwen3 GGUF exists in this environment, so the end-to-end gate
(|delta logprob| <= 2.7e-5 between the reference's attention and this build's) is measured on a
synthetic model with the Qwen3 block structure of src/model.cpp:157-236:

    h   = rmsnorm(x) * attn_norm                       (src/model.cpp:167)
    qkv = h @ [Wq; Wk; Wv]^T                            (:170-172)
    per-head QK-norm + RoPE, KV append, attention       (:174-214)  <- the path under test
    x  += att @ Wo^T                                    (:216)
    h   = rmsnorm(x) * ffn_norm; x += (silu(h Wg^T) * (h Wu^T)) Wd^T   (:218-230)
    logits = rmsnorm(x) * out_norm @ Wlm^T              (:233-236)

Everything except the attention callback is shared numpy float32 code, so two runs differ only
by how the attention sub-step (norm, RoPE, append, softmax attention) is computed.
"""
from __future__ import annotations

import numpy as np

HEAD_DIM = 128


def _rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    inv = (1.0 / np.sqrt(ss / x.shape[-1] + eps)).astype(np.float32)
    return (x * inv) * w


def _silu(x: np.ndarray) -> np.ndarray:
    return x / (1.0 + np.exp(-x))


class TinyQwen3:
    """Random Qwen3-shaped weights (head_dim 128); fan-in scaled so activations stay O(1)."""

    def __init__(self, seed: int, n_layer: int = 2, n_embd: int = 256, n_head: int = 4, n_head_kv: int = 2,
                 n_ff: int = 512, n_vocab: int = 384):
        rng = np.random.default_rng(seed)
        D = HEAD_DIM
        self.n_layer, self.E, self.H, self.HKV, self.V = n_layer, n_embd, n_head, n_head_kv, n_vocab

        def mat(rows, cols, gain=1.0):
            return (rng.standard_normal((rows, cols)) * (gain / np.sqrt(cols))).astype(np.float32)

        def norm_w(n):
            return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)

        self.emb = rng.standard_normal((n_vocab, n_embd)).astype(np.float32)
        self.layers = []
        for _ in range(n_layer):
            self.layers.append(dict(
                attn_norm=norm_w(n_embd),
                wqkv=mat((n_head + 2 * n_head_kv) * D, n_embd),
                q_norm=norm_w(D), k_norm=norm_w(D),
                wo=mat(n_embd, n_head * D),
                ffn_norm=norm_w(n_embd),
                wg=mat(n_ff, n_embd), wu=mat(n_ff, n_embd), wd=mat(n_embd, n_ff),
            ))
        self.out_norm = norm_w(n_embd)
        self.lm = mat(n_vocab, n_embd, gain=2.0)

    @classmethod
    def from_gguf(cls, path, dequant=None) -> "TinyQwen3":
        """The model a GGUF file holds, read through this build's C++ reader (exactinfer_amd.gguf):
        configuration and tensor table validated as read_config / read_tensors do
        (src/model.cpp:38-103); F16 matrices widened to float32 exactly.  Quantised tensors are
        decoded with dequant(type, blocks, n) (the oracle's decode of the reference's formats), and
        the attention projections also keep their raw bytes (layer key "qkv_raw": (type, blocks)
        of Wq, Wk, Wv) for a projection that reads the blocks themselves."""
        from exactinfer_amd.gguf import GgufFile
        self = cls.__new__(cls)
        D = HEAD_DIM
        with GgufFile(path) as g:
            c = g.qwen3_config()
            if c["head_dim"] != D or c["rope_dim"] != D:
                raise ValueError("the harness is built for head_dim = rope_dim = 128")

            def t(n):
                a = g.tensor(n)
                ty, ne, _ = g.tensor_info(n)
                if ty in (0, 1):
                    return np.ascontiguousarray(a, dtype=np.float32)
                if dequant is None:
                    raise ValueError(f"{n}: quantised (type {ty}) and no dequant given")
                return dequant(ty, a, ne[0]).reshape(a.shape[0], ne[0])

            def raw(n):
                ty = g.tensor_info(n)[0]
                a = g.tensor(n)
                return ty, (a.view(np.uint16) if ty == 1 else np.ascontiguousarray(a))
            self.n_layer, self.E, self.H, self.HKV, self.V = (c["n_layer"], c["n_embd"], c["n_head"], c["n_head_kv"],
                                                              c["n_vocab"])
            self.emb = t("token_embd.weight")
            self.out_norm = t("output_norm.weight")
            self.lm = t("output.weight") if g.tensor_info("output.weight") else self.emb
            self.layers = []
            for l in range(self.n_layer):
                b = f"blk.{l}."
                self.layers.append(dict(
                    attn_norm=t(b + "attn_norm.weight"),
                    wqkv=np.concatenate([t(b + "attn_q.weight"), t(b + "attn_k.weight"), t(b + "attn_v.weight")]),
                    qkv_raw=[raw(b + "attn_q.weight"), raw(b + "attn_k.weight"), raw(b + "attn_v.weight")],
                    q_norm=t(b + "attn_q_norm.weight"), k_norm=t(b + "attn_k_norm.weight"),
                    wo=t(b + "attn_output.weight"), ffn_norm=t(b + "ffn_norm.weight"),
                    wg=t(b + "ffn_gate.weight"), wu=t(b + "ffn_up.weight"), wd=t(b + "ffn_down.weight")))
        return self

    @property
    def qkv_width(self) -> int:
        return (self.H + 2 * self.HKV) * HEAD_DIM

    def forward(self, tokens: np.ndarray, pos0: int, attn, project=None) -> np.ndarray:
        """Logits [n, vocab] for tokens at positions pos0.. ; attn(l, qkv [n, qkv_width], pos0) -> [n, H*128].
        project(l, x) -> qkv [n, qkv_width], when given, replaces the attention RMSNorm + QKV product."""
        x = self.emb[tokens]
        for l, L in enumerate(self.layers):
            if project is not None:
                qkv = np.ascontiguousarray(project(l, x), dtype=np.float32)
            else:
                h = _rmsnorm(x, L["attn_norm"])
                qkv = np.ascontiguousarray(h @ L["wqkv"].T, dtype=np.float32)
            att = attn(l, qkv, pos0)
            x = x + att @ L["wo"].T
            h = _rmsnorm(x, L["ffn_norm"])
            x = x + (_silu(h @ L["wg"].T) * (h @ L["wu"].T)) @ L["wd"].T
        return _rmsnorm(x, self.out_norm) @ self.lm.T


def logprobs(logits: np.ndarray, targets: np.ndarray) -> np.ndarray:
    """log softmax(logits)[target] per row, evaluated in float64 from the float32 logits."""
    z = logits.astype(np.float64)
    z = z - z.max(axis=-1, keepdims=True)
    lse = np.log(np.exp(z).sum(axis=-1))
    return z[np.arange(len(targets)), targets] - lse


def run_sequence(model: TinyQwen3, attn_factory, tokens: np.ndarray, chunks: list[int], n_decode: int,
                 n_ctx: int, project=None) -> np.ndarray:
    """Prompt in `chunks` (prefill), then `n_decode` greedy-free decode steps on the given tokens.

    `tokens` holds sum(chunks) + n_decode + 1 ids; the logprob of token i+1 is scored at every
    position i.  attn_factory(n_ctx) returns the attention callback with its own KV cache.
    """
    attn = attn_factory(n_ctx)
    out = []
    pos = 0
    for n in chunks:
        lg = model.forward(tokens[pos:pos + n], pos, attn, project)
        out.append(logprobs(lg, tokens[pos + 1:pos + n + 1]))
        pos += n
    for _ in range(n_decode):
        lg = model.forward(tokens[pos:pos + 1], pos, attn, project)
        out.append(logprobs(lg, tokens[pos + 1:pos + 2]))
        pos += 1
    return np.concatenate(out)


def oracle_attention(model: TinyQwen3, O, scale: float | None = None, f64: bool = False):
    """Attention callback built on the CPU restatement (oracle/oracle.py) with per-layer caches."""
    D, H, HKV = HEAD_DIM, model.H, model.HKV

    def factory(n_ctx: int):
        kc = [np.zeros((n_ctx, HKV * D), np.float32) for _ in range(model.n_layer)]
        vc = [np.zeros((n_ctx, HKV * D), np.float32) for _ in range(model.n_layer)]

        def attn(l, qkv, pos0):
            L = model.layers[l]
            buf = O.headnorm_rope(qkv, H, D, L["q_norm"], pos0, D, 1e6, 1e-6)  # returns a normed copy
            buf = O.headnorm_rope(buf, HKV, D, L["k_norm"], pos0, D, 1e6, 1e-6, col0=H * D)
            O.kv_append(buf[:, H * D:(H + HKV) * D], buf[:, (H + HKV) * D:], kc[l], vc[l], pos0)
            n = buf.shape[0]
            q = np.ascontiguousarray(buf[:, :H * D])
            if f64:
                rows = [O.attn_f64(q[b].reshape(H, D), kc[l], vc[l], pos0 + b + 1, H, HKV, D, scale)
                        for b in range(n)]
                return np.stack(rows).reshape(n, H * D).astype(np.float32)
            if n == 1:
                return O.attn_decode(q.reshape(H, D), kc[l], vc[l], pos0 + 1, H, HKV, D, scale).reshape(1, H * D)
            return O.attn_prefill(q, kc[l], vc[l], n, pos0, H, HKV, D, scale).reshape(n, H * D)

        return attn

    return factory


def greedy_generate(model: TinyQwen3, attn, prompt: np.ndarray, n: int, chunk: int, start: int = 0):
    """The reference's generate/serve loop (src/main.cpp:497-531) on one attention instance:
    evaluate prompt[start:] in chunks of `chunk` at positions start.. (rows [0, start) of the
    caches are reused as they are), then n greedy steps.  Returns (tokens, logprobs of them)."""
    pos = start
    logits = None
    while pos < len(prompt):
        b = min(chunk, len(prompt) - pos)
        logits = model.forward(prompt[pos:pos + b], pos, attn)
        pos += b
    toks, lps = [], []
    last = logits[-1]
    for _ in range(n):
        z = last.astype(np.float64)
        nxt = int(np.argmax(z))
        zz = z - z.max()
        lps.append(float(zz[nxt] - np.log(np.exp(zz).sum())))
        toks.append(nxt)
        last = model.forward(np.array([nxt]), pos, attn)[-1]
        pos += 1
    return toks, np.array(lps)


class PrefixServer:
    """Serve mode (src/main.cpp:497-531): one persistent attention instance; a request reuses
    the cache rows of its longest common prefix with the cached tokens and re-evaluates at
    least its last prompt token."""

    def __init__(self, model: TinyQwen3, attn_factory, n_ctx: int, chunk: int):
        self.model, self.attn, self.chunk = model, attn_factory(n_ctx), chunk
        self.cached: list[int] = []

    def request(self, prompt: np.ndarray, n: int):
        common = 0
        while common < min(len(self.cached), len(prompt)) and self.cached[common] == int(prompt[common]):
            common += 1
        start = min(common, len(prompt) - 1)
        toks, lps = greedy_generate(self.model, self.attn, prompt, n, self.chunk, start)
        self.cached = [int(t) for t in prompt] + toks[:-1]  # the last generated token is not evaluated
        return toks, lps, start


def oracle_projection(model: TinyQwen3, O):
    """project(l, x) of the reference's CPU path on the file's own weights: rmsnorm
    (src/ops.cpp:155-160), then matvec of Wq, Wk, Wv as stored (dot_f32 / dot_f16, or the
    quantised decode + dot_f32; src/ops.cpp:126-153)."""
    def project(l, x):
        L = model.layers[l]
        rows = []
        for b in range(x.shape[0]):
            h = O.rmsnorm(np.ascontiguousarray(x[b], dtype=np.float32), L["attn_norm"])
            rows.append(np.concatenate([O.matvec(w, h, ty) for ty, w in L["qkv_raw"]]))
        return np.stack(rows)
    return project
