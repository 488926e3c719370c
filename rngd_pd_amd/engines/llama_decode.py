"""The full Llama decode step on MI355X: one token for each of B streams.

Replaces the reference's BatchDecodeEngine.step / step_logits
(engines/decode_batch.py:422-442) and its compiled DecodeLayer
(kernels/decode_batch.py:56-91) plus the batched lm_head and greedy argmax
(engines/decode_batch.py:162-171). The two RMSNorms of a layer and the final
one have no launch of their own: rmsnorm(x) . W^T = r * (x . (W diag g)^T)
with r = rsqrt(mean(x^2) + eps) per row, so each norm's gain g is folded into
the columns of the weights that follow it (once, when the decoder is built),
the kernel that produces x also writes its per-16-column sums of squares
(ssq), and the kernel that consumes the projection scales each row by r. Per
layer, one launch per line:

  qkv halves = r x . (Wqkv diag g1)^T              pdk_linear_splitk_rms (fp32 halves of K, rows scaled)
  q, k, v = bf16(sum of halves); RoPE(q, k); new
  k, v into the paged cache; ao = attention        pdk_decode_attn_rope (+ its merge when split)
  x = x + ao . Wo^T; ssq                            pdk_linear_ssq, residual fused
  a = silu(r g) * (r u), [g; u] = x . (Wgu diag g2)^T  pdk_linear_swiglu_rms
  x = x + a . Wd^T; ssq                             pdk_linear_ssq, residual fused

before the first layer pdk_embed_ssq gathers the embedding rows and writes
their ssq, and after the last the lm_head GEMM (weights folded with the final
norm's gain) scales each row's logits by r and takes the first-maximum argmax
in its epilogue (pdk_linear_argmax_rms).
Weights are [out, in] contiguous (torch Linear layout) with q|k|v and gate|up
stacked, so each projection is one pass over its weights. By default the
decoder streams tiled copies of them (pdk_weight_tile, made once at
construction: each 16-row x 128-column block contiguous in the order the GEMM
reads it) through the *_tiled entry points, with bit-identical results, and
keeps the activations (the residual stream, attention's output and SwiGLU's
output) in the matching tiled layout (act_tile; the *_xt entry points), so
each GEMM reads its activation operand 1 KiB at a time as well.
Activations are bf16 at every tensor boundary, as the reference's are; the
kernels accumulate in fp32 and round once.
"""
import contextlib
import math

import torch

from .. import _lib
from ..kernels import attention as _attn
from ..kernels.decode_step import act_rows, act_untile, fold_norm, tile_weight
from ..kernels.handoff import stream_handle

BF16 = torch.bfloat16


class LlamaConfig:
    """Llama-3.1-8B by default (engines/model.py:14-31 reads these from the HF config)."""

    def __init__(self, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, inter=14336,
                 vocab=128256, n_layers=32, eps=1e-5, theta=500000.0,
                 rope_scaling=(8.0, 1.0, 4.0, 8192)):
        self.hidden, self.n_heads, self.n_kv_heads, self.head_dim = hidden, n_heads, n_kv_heads, head_dim
        self.inter, self.vocab, self.n_layers, self.eps = inter, vocab, n_layers, eps
        self.theta = theta
        self.rope_scaling = rope_scaling   # (factor, low_freq_factor, high_freq_factor, original_max_pos) or None

    @property
    def qkv_dim(self):
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim

    def inv_freq(self):
        """float32 [head_dim/2]: theta^(-2i/d), with the llama3 band scaling
        (engines/model.py:32-48): long wavelengths divided by `factor`, short ones
        kept, the band between interpolated."""
        d = self.head_dim
        inv = [1.0 / (self.theta ** (2 * i / d)) for i in range(d // 2)]
        if self.rope_scaling:
            factor, lo, hi, orig = self.rope_scaling
            low_wl, high_wl = orig / lo, orig / hi
            out = []
            for f in inv:
                wl = 2 * math.pi / f
                if wl > low_wl:
                    out.append(f / factor)
                elif wl < high_wl:
                    out.append(f)
                else:
                    s = (orig / wl - lo) / (hi - lo)
                    out.append((1 - s) * f / factor + s * f)
            inv = out
        return torch.tensor(inv, dtype=torch.float64).to(torch.float32)


class LlamaWeights:
    """Decode-step weights, [out, in] contiguous bf16 on one device: wqkv
    [L, (NH + 2 NKV) HD, H], wo [L, H, NH HD], wgu [L, 2M, H] (gate rows then
    up rows), wd [L, H, M], embed [V, H], lm_head [V, H]."""

    def __init__(self, cfg, norm1, wqkv, wo, norm2, wgu, wd, embed, norm_f, lm_head):
        self.cfg = cfg
        self.norm1, self.wqkv, self.wo, self.norm2 = norm1, wqkv, wo, norm2
        self.wgu, self.wd = wgu, wd
        self.embed, self.norm_f, self.lm_head = embed, norm_f, lm_head

    @classmethod
    def random(cls, cfg, seed=0, device="cuda", std=0.02):
        """Random-init weights of the given shape (no checkpoint is fetched):
        projections N(0, std), norms 1 + N(0, 0.05), embedding N(0, 1)."""
        g = torch.Generator(device=device).manual_seed(seed)
        L, H, M = cfg.n_layers, cfg.hidden, cfg.inter

        def w(*shape, scale=std, mean=0.0):
            return (torch.randn(shape, generator=g, device=device) * scale + mean).to(BF16)

        return cls(cfg,
                   norm1=w(L, H, scale=0.05, mean=1.0),
                   wqkv=w(L, cfg.qkv_dim, H),
                   wo=w(L, H, cfg.n_heads * cfg.head_dim),
                   norm2=w(L, H, scale=0.05, mean=1.0),
                   wgu=w(L, 2 * M, H),
                   wd=w(L, H, M),
                   embed=w(cfg.vocab, H, scale=1.0),
                   norm_f=w(H, scale=0.05, mean=1.0),
                   lm_head=w(cfg.vocab, H))

    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in
                   (self.norm1, self.wqkv, self.wo, self.norm2, self.wgu, self.wd, self.embed,
                    self.norm_f, self.lm_head))


class LlamaDecoder:
    """B-stream decode steps over a PagedKVCache (same n_layers, Hkv, head_dim)."""

    def __init__(self, weights, cache, max_batch, tiled=True, plan_batch=None):
        """``tiled``: stream tiled copies of the projection and lm_head weights
        (the copies take as much device memory as those weights again; the
        originals are left untouched). ``plan_batch`` (default max_batch): the
        batch size every step's attention plans its context split for. Each
        stream's result then does not depend on how many streams share a step:
        every other kernel of the step computes a row independently of the
        others, so a stream's tokens are the same at B = 1 as in any batch of
        a decoder with the same plan_batch."""
        cfg = self.cfg = weights.cfg
        if (cache.n_layers, cache.n_kv_heads, cache.head_dim) != (cfg.n_layers, cfg.n_kv_heads,
                                                                  cfg.head_dim):
            raise ValueError("cache shape does not match the model")
        self.w, self.cache = weights, cache
        dev = self.device = cache.k.device          # the real device (cuda:N)
        B, H = max_batch, cfg.hidden
        self.max_batch = B
        self.plan_batch = int(plan_batch or max_batch)
        if self.plan_batch < max_batch:
            raise ValueError(f"plan_batch={plan_batch} below max_batch={max_batch}")
        self._captured = False
        e = lambda *s: torch.empty(s, dtype=BF16, device=dev)   # noqa: E731
        # Activations (the residual stream x, attention's output, SwiGLU's
        # output) in the tiled layout the GEMMs read as their MFMA operand
        # (act_tile; the _xt entry points) when the weights are tiled and every
        # width is a multiple of 128, else row-major [B, .].
        self.act_tiled = bool(tiled) and cfg.inter % 16 == 0 and all(
            d % 128 == 0 for d in (H, cfg.inter, cfg.n_heads * cfg.head_dim))
        if self.act_tiled:
            rows = act_rows(B)
            self.x_buf = e(rows * H)
            self.ao = e(rows * cfg.n_heads * cfg.head_dim)
            self.act = e(rows * cfg.inter)
        else:
            self.x_buf = e(B, H)
            self.ao = e(B, cfg.n_heads, cfg.head_dim)
            self.act = e(B, cfg.inter)
        self.logits = e(B, cfg.vocab)
        self.tokens = torch.empty(B, dtype=torch.int32, device=dev)
        self.keys = torch.zeros(B, dtype=torch.int64, device=dev)    # argmax scratch, kept zero
        # The down projection (K = 14336 at 8B) runs as the O projection does:
        # one workgroup per 16 columns over all of K, residual and sums of
        # squares in its epilogue. Split over K in two with 32 columns per
        # workgroup (pdk_linear_splitk_final: half the activation re-reads,
        # and the last split of each column group adds the partials) the
        # 8B step took as long at B = 16 (2.923-2.925 against 2.920-2.927 ms)
        # and 34 us longer at B = 4 (2.767-2.770 against 2.733-2.738), in one
        # process with step-major tiled weights.
        # The q|k|v projection (N = 6144 at 8B) splits K in two when every wave
        # of the GEMM still gets two 128-long steps of each half: 2 x 96 wide
        # workgroups instead of 384 narrow ones, which re-read x per 16
        # columns. The attention kernel adds the halves (and applies RoPE).
        self.qkv_splits = 2 if H // 128 >= 32 else 1
        self.part_qkv = torch.empty((self.qkv_splits, B, cfg.qkv_dim), dtype=torch.float32,
                                    device=dev)
        # Per 16-column tile and row, the residual's sums of squares: left by
        # the O projection for the post-attention norm (fused into gate|up),
        # and by the down projection (pdk_embed_ssq before layer 0) for the
        # pre-attention norm (fused into attention) and the final one (into
        # the lm_head).
        self.ssq = torch.zeros((B, H // 16), dtype=torch.float32, device=dev)
        self.ssq_a = torch.zeros((B, H // 16), dtype=torch.float32, device=dev)
        self.inv = cfg.inv_freq().to(dev)
        self.scale = 1.0 / math.sqrt(cfg.head_dim)
        self._ws = None
        # Per-layer operands resolved once: the step loop makes no views.
        w = weights
        if max_batch > 64:
            raise ValueError("the decode GEMMs take at most 64 streams")
        # Tiled copies need M % 16 == 0 for gate|up and K % 128 == 0 (as the
        # GEMMs themselves do).
        self.tiled = bool(tiled) and cfg.inter % 16 == 0
        prep = tile_weight if self.tiled else (lambda t: t)
        # q|k|v, gate|up and the lm_head with their norms' gains folded into
        # their columns (copies in either layout; the originals stay as they
        # are).
        self._wt = [(prep(fold_norm(w.wqkv[i], w.norm1[i])), prep(w.wo[i]),
                     prep(fold_norm(w.wgu[i], w.norm2[i])), prep(w.wd[i]))
                    for i in range(cfg.n_layers)]
        self._lm_head = prep(fold_norm(w.lm_head, w.norm_f))
        if self.tiled:
            # The copies are written on the current stream; a step may run on
            # another one, so they are complete before the constructor returns.
            torch.cuda.current_stream(dev).synchronize()
        suffix = "_xt" if self.act_tiled else "_tiled" if self.tiled else ""
        self._gemm = {n: n + suffix for n in
                      ("pdk_linear_splitk_rms", "pdk_linear_ssq", "pdk_linear_swiglu_rms",
                       "pdk_linear_argmax_rms")}
        self._gemm["pdk_embed_ssq"] = "pdk_embed_ssq_xt" if self.act_tiled else "pdk_embed_ssq"
        self._gemm["pdk_decode_attn_rope"] = ("pdk_decode_attn_rope_xt" if self.act_tiled
                                              else "pdk_decode_attn_rope")
        if cfg.hidden % 16 or cfg.head_dim != 128:
            raise ValueError("the fused norms need hidden % 16 == 0 and head_dim 128")
        self._layers = [tuple(t.data_ptr() for t in (wt[0], wt[1], wt[2], wt[3], cache.k[i],
                                                     cache.v[i]))
                        for i, wt in enumerate(self._wt)]

    @property
    def x(self):
        """The residual stream [max_batch, hidden] (bf16), row-major: after a
        step, rows :B hold the final hidden state before the final norm. A
        copy when the decoder keeps it tiled (x_buf is the buffer itself)."""
        if self.act_tiled:
            return act_untile(self.x_buf, self.max_batch, self.cfg.hidden)
        return self.x_buf

    def reserve(self, max_ctx):
        """Allocate the attention workspace for max_batch streams at ``max_ctx``
        now, so that no later step (or graph capture) allocates it."""
        self._workspace(self.plan_batch, max_ctx)

    def _workspace(self, B, max_ctx):
        """The attention workspace, grown when a step needs more. A captured
        graph holds the address it was captured with, so once any graph exists
        a step that would need a larger one raises instead (reserve() the
        largest max_ctx before capturing)."""
        need = _attn.workspace_bytes(B, self.cfg.n_heads, max_ctx, self.cfg.head_dim)
        if need and (self._ws is None or self._ws.numel() * 4 < need):
            if self._captured:
                raise RuntimeError(f"the attention workspace would have to grow to {need} bytes "
                                   f"after a graph was captured with the old one; reserve() the "
                                   f"largest max_ctx before capturing")
            self._ws = torch.zeros(need // 4 + 64, dtype=torch.float32, device=self.device)
        return self._ws if need else None

    def step(self, tokens, ctx_lens, tables, max_ctx, stream=None):
        """tokens int64/int32 [B] on the device (this step's input token per
        stream; an id outside [0, vocab) embeds as a zero row), ctx_lens int32 [B] = position + 1 (the new token's slot is
        ctx_lens-1, attention covers 0..ctx_lens-1), tables int32 [B, max_blocks]
        holding at least ceil(ctx/16) blocks each; max_ctx (<= max_blocks*16)
        sizes the attention's split plan and should cover every ctx_lens. Returns
        the next token per stream (int32 [B], device) and leaves the final hidden
        state in rows :B of the residual stream (self.x, before the final norm)
        and the logits in self.logits[:B]. ``stream``: a torch stream for every launch (default:
        the current stream)."""
        cfg, w, cache = self.cfg, self.w, self.cache
        B = tokens.shape[0]
        if B > self.max_batch:
            raise ValueError(f"B={B} above max_batch={self.max_batch}")
        for t, name in ((tokens, "tokens"), (ctx_lens, "ctx_lens"), (tables, "tables")):
            if not t.is_cuda or t.device != self.device:
                raise ValueError(f"{name} must be on {self.device}")
        if tokens.dtype not in (torch.int32, torch.int64) or tokens.dim() != 1 \
                or not tokens.is_contiguous():
            raise ValueError("tokens must be contiguous int32 or int64 [B]")
        if ctx_lens.dtype != torch.int32 or ctx_lens.numel() != B:
            raise ValueError("ctx_lens must be int32 [B]")
        if tables.dtype != torch.int32 or tables.dim() != 2 or tables.shape[0] != B \
                or not tables.is_contiguous():
            raise ValueError("tables must be contiguous int32 [B, max_blocks]")
        st = stream_handle(stream)
        H, NH, NKV, HD, M = cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.inter
        QKV, eps = cfg.qkv_dim, cfg.eps
        ws = self._workspace(max(B, self.plan_batch), max_ctx)
        ws_ptr = ws.data_ptr() if ws is not None else None
        ws_bytes = ws.numel() * 4 if ws is not None else 0
        mb, nb = tables.shape[1], cache.num_blocks
        tp, cp = tables.data_ptr(), ctx_lens.data_ptr()
        xp = self.x_buf.data_ptr()
        aop, actp, inv = self.ao.data_ptr(), self.act.data_ptr(), self.inv.data_ptr()
        call = _lib.call
        g = self._gemm
        lin_skr = g["pdk_linear_splitk_rms"]
        lin_ssq, lin_swr, lin_amr = (g["pdk_linear_ssq"], g["pdk_linear_swiglu_rms"],
                                     g["pdk_linear_argmax_rms"])
        ssqp, ssqa, n_ssq = self.ssq.data_ptr(), self.ssq_a.data_ptr(), H // 16
        emb, attn = g["pdk_embed_ssq"], g["pdk_decode_attn_rope"]
        with torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext():
            call(emb, w.embed.data_ptr(), cfg.vocab, tokens.data_ptr(),
                 tokens.element_size(), B, H, xp, ssqa, st)
            pqp, qs = self.part_qkv.data_ptr(), self.qkv_splits
            for wqkv, wo, wgu, wd, ck, cv in self._layers:
                call(lin_skr, xp, wqkv, B, H, QKV, qs, ssqa, n_ssq, eps, pqp, st)
                call(attn, pqp, qs, inv, ck, cv, nb, tp, mb, cp, int(max_ctx),
                     B, NH, NKV, HD, self.scale, ws_ptr, ws_bytes, aop, self.plan_batch, st)
                call(lin_ssq, aop, wo, B, NH * HD, H, xp, xp, ssqp, st)
                call(lin_swr, xp, wgu, B, H, M, ssqp, n_ssq, eps, actp, st)
                call(lin_ssq, actp, wd, B, M, H, xp, xp, ssqa, st)
            call(lin_amr, xp, self._lm_head.data_ptr(), B, H, cfg.vocab, ssqa, n_ssq, eps,
                 self.logits.data_ptr(), self.keys.data_ptr(), self.tokens.data_ptr(), st)
        return self.tokens[:B]

    def capture(self, tokens, ctx_lens, tables, max_ctx):
        """One step captured as a HIP graph over these device tensors.

        replay() re-runs the step on whatever tokens, ctx_lens and tables hold
        then (the caller updates them in place; max_ctx is fixed at capture, so
        pass the tables' capacity to allow any context). One warm step runs
        first, eagerly, on the capture stream: it is a real step (it writes the
        cache slot of each stream's current position)."""
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self.step(tokens, ctx_lens, tables, max_ctx)
        torch.cuda.current_stream(self.device).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        # Thread-local capture: other threads of the process (cache loaders)
        # may synchronise on their own streams while this one captures.
        self._captured = True
        with torch.cuda.graph(graph, capture_error_mode="thread_local"):
            self.step(tokens, ctx_lens, tables, max_ctx)
        return graph
