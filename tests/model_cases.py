"""Shared builders for the model-level tests: a synthetic GGUF model, its LoRA adapters, and the
oracle's description of the same model (tensors read back from the GGUF image)."""
import numpy as np

import oracle as O
from rust_trainer_amd import gguf as G

GGUF_NAMES = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate", "up": "ffn_up",
              "down": "ffn_down"}


def tiny_spec(wtype, n_layer=2, arch="qwen3", tied=True, **kw):
    s = G.SyntheticSpec.tiny(arch, wtype)
    s.n_layer = n_layer
    s.tied_output = tied
    for k, v in kw.items():
        setattr(s, k, v)
    return s


def adapters(g: G.GgufFile, rank: int, alpha: float, seed: int = 11, b_std: float = 0.01):
    """{(layer, linear): (A [r x in], B [out x r])}: A as Lora::new draws it (uniform in
    +-1/sqrt(in)), B ~ N(0, b_std) (non-zero, so both adapter paths carry gradient)."""
    rng = O.Rng(seed)
    n_layer = g.get_u32(f"{g.get_str('general.architecture')}.block_count")
    out = {}
    for li in range(n_layer):
        for name, gname in GGUF_NAMES.items():
            t = g.tensor(f"blk.{li}.{gname}.weight")
            A = rng.vec_uniform_sym(rank * t.row_len(), 1.0 / np.sqrt(t.row_len())).reshape(rank, t.row_len())
            B = rng.vec_normal(t.n_rows() * rank, b_std).reshape(t.n_rows(), rank)
            out[(li, name)] = (A.astype(np.float32), B.astype(np.float32))
    return out


def oracle_model(g: G.GgufFile, lora=None, alpha=0.0, kv_f16=True):
    arch = g.get_str("general.architecture")
    n_layer = g.get_u32(f"{arch}.block_count")

    def W(name):
        t = g.tensor(name)
        return dict(wtype=t.ty, blocks=np.array(g.tensor_data(t)), out=t.n_rows(), **{"in": t.row_len()})

    def vec(name):
        t = g.tensor(name)
        return None if t is None else g.tensor_f32(t).reshape(-1)

    layers = []
    for li in range(n_layer):
        p = f"blk.{li}."
        ld = dict(attn_norm=vec(p + "attn_norm.weight"), ffn_norm=vec(p + "ffn_norm.weight"),
                  q_norm=vec(p + "attn_q_norm.weight"), k_norm=vec(p + "attn_k_norm.weight"))
        for name, gname in GGUF_NAMES.items():
            ld[name] = W(p + gname + ".weight")
            if lora is not None and (li, name) in lora:  # linears missing from lora are not adapted
                A, B = lora[(li, name)]
                ld[name].update(A=A, B=B, alpha=alpha)
        layers.append(ld)
    emb = g.tensor("token_embd.weight")
    head = g.tensor("output.weight") or emb
    hd = g.get_u32(f"{arch}.attention.key_length")
    return dict(n_layer=n_layer, d=g.get_u32(f"{arch}.embedding_length"), n_head=g.get_u32(f"{arch}.attention.head_count"),
                n_kv=g.get_u32(f"{arch}.attention.head_count_kv"), hd=hd,
                rot=g.get_u32(f"{arch}.rope.dimension_count") or hd, n_ff=g.get_u32(f"{arch}.feed_forward_length"),
                eps=g.get_f32(f"{arch}.attention.layer_norm_rms_epsilon"), off=0.0,
                theta=g.get_f32(f"{arch}.rope.freq_base"), freq_scale=1.0, neox=arch != "llama", kv_f16=kv_f16,
                embed=(emb.ty, np.array(g.tensor_data(emb)), emb.n_rows(), emb.row_len()),
                lm_head=(head.ty, np.array(g.tensor_data(head)), head.n_rows(), head.row_len()),
                out_norm=vec("output_norm.weight"), layers=layers)


def sequence(V: int, t: int, n: int, seed: int = 5):
    """t random token ids and answer targets on the last n positions (answer_targets)."""
    toks = (O.Rng(seed).vec_uniform_sym(t, 1.0) * 0.5 + 0.5) * (V - 1)
    toks = np.clip(np.rint(toks), 0, V - 1).astype(np.int32)
    start = t - n
    pos = np.arange(start - 1, t - 1, dtype=np.int32)
    tok = toks[start:t].copy()
    return toks, pos, tok
