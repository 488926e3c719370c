"""Pins of the decode-step oracle (oracle/decode.py) on the CPU.

The oracle restates the reference's cpu_layer; these checks tie it to things
it was not written from: transformers' own Llama (its llama3 RoPE init and
its full fp32 forward, run on the same weights), the reference's other RoPE
form (a per-stream [HD, HD] rotation matmul, kernels/decode_batch.py:111-122),
torch's rms_norm and silu, and invariants of the rotation.
"""
import math

import numpy as np
import pytest
import torch

from oracle import decode as od

LLAMA3 = (8.0, 1.0, 4.0, 8192)


def _hf_config(**kw):
    from transformers import LlamaConfig
    rp = {"rope_type": "llama3", "rope_theta": kw.pop("theta", 500000.0), "factor": LLAMA3[0],
          "low_freq_factor": LLAMA3[1], "high_freq_factor": LLAMA3[2],
          "original_max_position_embeddings": LLAMA3[3]}
    return LlamaConfig(rope_parameters=rp, max_position_embeddings=131072,
                       attn_implementation="eager", **kw)


@pytest.mark.parametrize("head_dim,theta", [(128, 500000.0), (64, 10000.0)])
def test_inv_freq_matches_transformers_llama3(head_dim, theta):
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    cfg = _hf_config(hidden_size=head_dim * 4, num_attention_heads=4, head_dim=head_dim,
                     theta=theta)
    want, _ = ROPE_INIT_FUNCTIONS["llama3"](cfg, "cpu")
    got = od.inv_freq(head_dim, theta, LLAMA3)
    np.testing.assert_allclose(got, want.numpy(), rtol=6e-7)   # float32 vs float64 then cast
    # All three bands occur at head_dim 128: divided, kept and interpolated.
    plain = od.inv_freq(head_dim, theta)
    ratio = got / plain
    if head_dim == 128:
        assert np.isclose(ratio, 1 / 8).any() and np.isclose(ratio, 1.0).any()
        assert ((ratio > 1 / 8 + 1e-3) & (ratio < 1 - 1e-3)).any()


def _rot_batch(inv, positions, HD):
    """The reference's rotation-matrix RoPE (kernels/decode_batch.py:111-122), restated."""
    half = HD // 2
    out = np.zeros((len(positions), HD, HD), np.float32)
    i = np.arange(half)
    for b, p in enumerate(positions):
        ang = np.float32(p) * inv
        cs, sn = np.cos(ang), np.sin(ang)
        out[b, i, i] = cs
        out[b, i + half, i + half] = cs
        out[b, i, i + half] = sn
        out[b, i + half, i] = -sn
    return out


def test_rope_equals_rotation_matmul_and_invariants():
    rng = np.random.default_rng(0)
    HD, B, nh = 128, 3, 5
    inv = od.inv_freq(HD, 500000.0, LLAMA3)
    t = rng.standard_normal((B, nh, HD)).astype(np.float32)
    positions = [0, 17, 4095]
    got = od.rope(t, positions, inv)
    rot = _rot_batch(inv, positions, HD)
    want = np.einsum("bnh,bhk->bnk", t, rot)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(got[0], t[0])                     # position 0 is the identity
    # Each (i, i + HD/2) pair keeps its length.
    pair = lambda x: x[..., :HD // 2] ** 2 + x[..., HD // 2:] ** 2   # noqa: E731
    np.testing.assert_allclose(pair(got), pair(t), rtol=1e-4, atol=1e-5)
    # q(m).k(n) depends only on m - n.
    q, k = t[:1, :1], t[1:2, :1]
    d1 = (od.rope(q, [40], inv) * od.rope(k, [30], inv)).sum()
    d2 = (od.rope(q, [110], inv) * od.rope(k, [100], inv)).sum()
    assert abs(d1 - d2) < 1e-3 * (abs(d1) + 1)


def test_rmsnorm_and_swiglu_match_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 512)).astype(np.float32) * 3
    w = rng.standard_normal(512).astype(np.float32)
    want = torch.nn.functional.rms_norm(torch.from_numpy(x), (512,), torch.from_numpy(w), 1e-5)
    np.testing.assert_allclose(od.rmsnorm(x, w, 1e-5), want.numpy(), rtol=1e-5, atol=1e-6)
    gu = rng.standard_normal((4, 2 * 96)).astype(np.float32) * 4
    t = torch.from_numpy(gu)
    want = torch.nn.functional.silu(t[:, :96]) * t[:, 96:]
    np.testing.assert_allclose(od.swiglu(gu), want.numpy(), rtol=1e-5, atol=1e-6)


def test_attention_masks_after_position():
    """Slots after pos carry no weight: changing them changes nothing; the
    context of one slot returns that slot's V."""
    rng = np.random.default_rng(2)
    B, NH, NKV, S, HD = 2, 4, 2, 9, 16
    q = rng.standard_normal((B, NH, HD)).astype(np.float32)
    K = rng.standard_normal((B, NKV, S, HD)).astype(np.float32)
    V = rng.standard_normal((B, NKV, S, HD)).astype(np.float32)
    out = od.attention(q, K, V, [3, 0])
    K2, V2 = K.copy(), V.copy()
    K2[:, :, 4:] += 100.0
    V2[:, :, 4:] -= 50.0
    np.testing.assert_allclose(od.attention(q, K2, V2, [3, 0]), out, rtol=1e-6)
    G = NH // NKV
    np.testing.assert_allclose(out[1], np.repeat(V[1, :, 0], G, axis=0), rtol=1e-6)


def _random_weights(rng, L, H, NH, NKV, HD, M, V):
    n = lambda *s, sc=0.05: (rng.standard_normal(s) * sc).astype(np.float32)   # noqa: E731
    layers = [(1 + n(H), n(H, (NH + 2 * NKV) * HD), n(NH * HD, H), 1 + n(H),
               n(H, 2 * M), n(M, H)) for _ in range(L)]
    return {"embed": n(V, H, sc=1.0), "layers": layers, "norm_f": 1 + n(H),
            "lm_head": n(H, V)}


class _Cfg:
    def __init__(self, n_heads, n_kv_heads, eps, inv):
        self.n_heads, self.n_kv_heads, self.eps, self.inv = n_heads, n_kv_heads, eps, inv


def test_decode_steps_match_transformers_llama_forward():
    """Token-by-token decode through the oracle (teacher forced, cache growing
    from empty) equals transformers' LlamaForCausalLM fp32 forward over the
    whole sequence at every position: hidden state after the final norm and
    logits, hence the greedy token too."""
    from transformers import LlamaForCausalLM
    L, H, NH, NKV, HD, M, V, T, B = 2, 256, 4, 2, 64, 384, 300, 10, 2
    eps = 1e-5
    rng = np.random.default_rng(3)
    w = _random_weights(rng, L, H, NH, NKV, HD, M, V)
    cfg = _hf_config(hidden_size=H, intermediate_size=M, num_attention_heads=NH,
                     num_key_value_heads=NKV, head_dim=HD, num_hidden_layers=L, vocab_size=V,
                     rms_norm_eps=eps, theta=500000.0)
    model = LlamaForCausalLM(cfg).float().eval()
    sd = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["norm_f"],
          "lm_head.weight": w["lm_head"].T}
    nq, nk = NH * HD, NKV * HD
    for i, (n1, wqkv, wo, n2, wgu, wd) in enumerate(w["layers"]):
        p = f"model.layers.{i}."
        sd.update({p + "input_layernorm.weight": n1, p + "post_attention_layernorm.weight": n2,
                   p + "self_attn.q_proj.weight": wqkv[:, :nq].T,
                   p + "self_attn.k_proj.weight": wqkv[:, nq:nq + nk].T,
                   p + "self_attn.v_proj.weight": wqkv[:, nq + nk:].T,
                   p + "self_attn.o_proj.weight": wo.T,
                   p + "mlp.gate_proj.weight": wgu[:, :M].T, p + "mlp.up_proj.weight": wgu[:, M:].T,
                   p + "mlp.down_proj.weight": wd.T})
    model.load_state_dict({k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sd.items()},
                          strict=True)
    ids = rng.integers(0, V, size=(B, T))
    with torch.no_grad():
        out = model(torch.from_numpy(ids), output_hidden_states=True)
    hf_hidden = out.hidden_states[-1].numpy()          # after the final norm
    hf_logits = out.logits.numpy()

    ocfg = _Cfg(NH, NKV, eps, od.inv_freq(HD, 500000.0, LLAMA3))
    Ks = [np.zeros((B, NKV, T, HD), np.float32) for _ in range(L)]
    Vs = [np.zeros((B, NKV, T, HD), np.float32) for _ in range(L)]
    for t in range(T):
        tok, x, logits = od.decode_step(ids[:, t], w, Ks, Vs, [t] * B, ocfg)
        np.testing.assert_allclose(od.rmsnorm(x, w["norm_f"], eps), hf_hidden[:, t],
                                   rtol=2e-4, atol=2e-4)
        np.testing.assert_allclose(logits, hf_logits[:, t], rtol=2e-4, atol=2e-4)
        np.testing.assert_array_equal(tok, hf_logits[:, t].argmax(-1))


def test_rel_l2():
    a = np.ones(100, np.float32)
    assert od.rel_l2(a, a) == 0.0
    assert math.isclose(od.rel_l2(a * 1.05, a), 0.05, rel_tol=1e-6)
