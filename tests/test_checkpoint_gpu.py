"""weights.Load through the library (tgohip_load_qwen3) on a Qwen3-shaped bf16
checkpoint written in Hugging Face's layout, against the same ports uploaded
one by one from numpy: decode (bf16 bits << 16), transpose [out, in] ->
[in, out], q/k head permutation y[2i] = x[i], y[2i+1] = x[i + d/2], then the
form's host conversion. A step over both contexts must give bit-identical
logits: the loader is a relabelling, so every weight on the device agrees to
the bit. Also the tied head and the loader's refusals."""
import os

import numpy as np
import pytest

import tgo_amd
from oracle import host
from stwrite import bf16_bits, write_arrays
from test_model_gpu import Engine, gpu_backend

pytestmark = pytest.mark.gpu

CFG = dict(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1024,
           eps=1e-6, theta=1e6, block=4, positions=256)


def checkpoint(tmp_path, seed, tie=False, drop=None, reshape=None):
    """Writes model.safetensors (bf16) and returns {tensor: f32 values it holds}."""
    rng = np.random.default_rng(seed)
    c = CFG
    d, qw, kvw, f, V, dh = (c["hidden"], c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"],
                            c["ffn"], c["vocab"], c["head_dim"])
    shapes = {"model.embed_tokens.weight": (V, d), "model.norm.weight": (d,)}
    if not tie:
        shapes["lm_head.weight"] = (V, d)
    for l in range(c["layers"]):
        p = "model.layers.%d." % l
        shapes.update({p + "input_layernorm.weight": (d,), p + "post_attention_layernorm.weight": (d,),
                       p + "self_attn.q_proj.weight": (qw, d), p + "self_attn.k_proj.weight": (kvw, d),
                       p + "self_attn.v_proj.weight": (kvw, d), p + "self_attn.o_proj.weight": (d, qw),
                       p + "self_attn.q_norm.weight": (dh,), p + "self_attn.k_norm.weight": (dh,),
                       p + "mlp.gate_proj.weight": (f, d), p + "mlp.up_proj.weight": (f, d),
                       p + "mlp.down_proj.weight": (d, f)})
    if reshape:
        shapes.update(reshape)
    arrays, values = {}, {}
    for name, shp in sorted(shapes.items()):
        if drop and name == drop:
            continue
        gain = len(shp) == 1
        x = (1.0 + 0.1 * rng.standard_normal(shp)) if gain else 0.02 * rng.standard_normal(shp)
        b = bf16_bits(x)
        arrays[name] = ("BF16", b)
        values[name] = (b.astype(np.uint32) << 16).view(np.float32)
    out = tmp_path / ("ckpt%d" % seed)
    out.mkdir()
    write_arrays(str(out / "model.safetensors"), arrays)
    return str(out), values


def permute(x, dh):
    s = x.reshape(-1, dh)
    return np.stack([s[:, : dh // 2], s[:, dh // 2:]], axis=-1).reshape(x.shape)


def upload_by_hand(ctx, values, form, tie):
    """The ports the loader should produce, from numpy."""
    c = CFG
    dh = c["head_dim"]

    def proj(port, w_out_in, f, heads_dim=0):
        w = np.ascontiguousarray(w_out_in.T)  # [in, out]
        if heads_dim:
            w = permute(w, heads_dim)
        K, N = w.shape
        if f == 0:
            h, _ = tgo_amd.to_f16(w)
            ctx.weight(port, 0, K, N, h)
        elif f == 1:
            q, s = tgo_amd.quantize_int8(w)
            ctx.weight(port, 1, K, N, q, s)
        else:
            cd, s, z = tgo_amd.quantize_int4(w)
            ctx.weight(port, 2, K, N, cd, s, z)

    emb = values["model.embed_tokens.weight"]
    ef = 0 if form == 0 else 1
    if ef == 0:
        h, _ = tgo_amd.to_f16(emb)
        ctx.weight("embed", 0, emb.shape[0], emb.shape[1], h)
    else:
        q, s = tgo_amd.quantize_int8(emb)
        ctx.weight("embed", 1, emb.shape[0], emb.shape[1], q, s)
    for l in range(c["layers"]):
        p = "model.layers.%d." % l
        ctx.gain("%d.attn_norm" % l, values[p + "input_layernorm.weight"])
        ctx.gain("%d.ffn_norm" % l, values[p + "post_attention_layernorm.weight"])
        ctx.gain("%d.qnorm" % l, permute(values[p + "self_attn.q_norm.weight"], dh))
        ctx.gain("%d.knorm" % l, permute(values[p + "self_attn.k_norm.weight"], dh))
        proj("%d.wq" % l, values[p + "self_attn.q_proj.weight"], form, dh)
        proj("%d.wk" % l, values[p + "self_attn.k_proj.weight"], form, dh)
        proj("%d.wv" % l, values[p + "self_attn.v_proj.weight"], form)
        proj("%d.wo" % l, values[p + "self_attn.o_proj.weight"], form)
        proj("%d.wgate" % l, values[p + "mlp.gate_proj.weight"], form)
        proj("%d.wup" % l, values[p + "mlp.up_proj.weight"], form)
        proj("%d.wdown" % l, values[p + "mlp.down_proj.weight"], form)
    ctx.gain("final_norm", values["model.norm.weight"])
    proj("lm_head", values["model.embed_tokens.weight" if tie else "lm_head.weight"], form)


def new_ctx(torch):
    c = CFG
    ctx = tgo_amd.Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    ctx.config(c["layers"], c["hidden"], c["heads"], c["kv_heads"], c["head_dim"], c["ffn"],
               c["vocab"], c["eps"], c["theta"], c["block"])
    return ctx


def run_steps(ctx):
    c = CFG
    ctx.kv_alloc(c["positions"])
    eng = Engine(gpu_backend(ctx), c["vocab"], c["heads"], c["kv_heads"], c["positions"],
                 c["block"], 3)
    rng = np.random.default_rng(11)
    prompts = [[int(t) for t in rng.integers(0, c["vocab"], n)] for n in (7, 20, 33)]
    for s, pr in enumerate(prompts):
        eng.admit(s, pr, reserve=8)
    out = [eng.step([(0, prompts[0]), (1, prompts[1][:12])])]
    out.append(eng.step([(1, prompts[1][12:]), (2, prompts[2]), (0, [5])]))
    return out


@pytest.mark.parametrize("form", [0, 1, 2])
@pytest.mark.parametrize("tie", [False, True])
def test_loaded_checkpoint_steps_bit_identical_to_ports_uploaded_by_hand(torch_gpu, tmp_path,
                                                                          form, tie):
    torch = torch_gpu
    path, values = checkpoint(tmp_path, 5, tie=tie)
    a = new_ctx(torch)
    with tgo_amd.Repo(path) as repo:
        sat = a.load_qwen3(repo, form, tie=tie)
    assert sat == 0
    b = new_ctx(torch)
    upload_by_hand(b, values, form, tie)
    la, lb = run_steps(a), run_steps(b)
    for x, y in zip(la, lb):
        assert np.isfinite(x).all()
        assert np.array_equal(x, y)
    a.close()
    b.close()


def test_loader_refusals(torch_gpu, tmp_path):
    torch = torch_gpu
    ctx = new_ctx(torch)
    path, _ = checkpoint(tmp_path, 1, drop="model.layers.1.mlp.up_proj.weight")
    with tgo_amd.Repo(path) as repo:
        with pytest.raises(tgo_amd.TgoError, match='declares "model.layers.1.mlp.up_proj.weight", '
                                                  'which this checkpoint does not contain'):
            ctx.load_qwen3(repo, 0)
    path, _ = checkpoint(tmp_path, 2, reshape={"model.layers.0.self_attn.k_proj.weight": (128, 256)})
    with tgo_amd.Repo(path) as repo:
        with pytest.raises(tgo_amd.TgoError, match=r"has shape \[128 256\] and the config declares "
                                                  r"\[256 256\]"):
            ctx.load_qwen3(repo, 0)
    path, _ = checkpoint(tmp_path, 3)  # ships lm_head.weight
    with tgo_amd.Repo(path) as repo:
        with pytest.raises(tgo_amd.TgoError, match="also ships"):
            ctx.load_qwen3(repo, 0, tie=True)
        with pytest.raises(tgo_amd.TgoError, match="int4 pack tgo stores"):
            ctx.load_qwen3(repo, 3)
    ctx.close()
