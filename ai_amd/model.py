"""Qwen3 checkpoints for the end-to-end harness: architecture configs, a
deterministic random initialisation, and a reader with the reference loader's
interface (ramvi/engine/ramvi_engine/formats/model.py:37-106).

No checkpoint can be downloaded here, so the models are random: every linear
and the embedding are bf16 N(0, 0.02), every RMSNorm weight is 1 (the Hugging
Face initialisation; N(0, 0.02) norms would shrink the logits and make greedy
ties likely).  Each tensor is drawn from its own generator seeded by
(model seed, tensor name), so any tensor can be regenerated on its own, bit
for bit (on the same generating device).

    ck = RandomCkpt(QWEN3["0.6b"], seed=0)     # tensors made on demand
    write_checkpoint(ck, "dir")                # config.json + model.safetensors
    ck2 = Ckpt("dir")                          # the same tensors, read back
"""
import json
import os
import zlib

import torch

QWEN3 = {
    "0.6b": dict(hidden_size=1024, num_hidden_layers=28, num_attention_heads=16, num_key_value_heads=8,
                 head_dim=128, intermediate_size=3072, vocab_size=151936, tie_word_embeddings=True,
                 rms_norm_eps=1e-6, rope_theta=1e6),
    "8b": dict(hidden_size=4096, num_hidden_layers=36, num_attention_heads=32, num_key_value_heads=8,
               head_dim=128, intermediate_size=12288, vocab_size=151936, tie_word_embeddings=False,
               rms_norm_eps=1e-6, rope_theta=1e6),
    "14b": dict(hidden_size=5120, num_hidden_layers=40, num_attention_heads=40, num_key_value_heads=8,
                head_dim=128, intermediate_size=17408, vocab_size=151936, tie_word_embeddings=False,
                rms_norm_eps=1e-6, rope_theta=1e6),
    "32b": dict(hidden_size=5120, num_hidden_layers=64, num_attention_heads=64, num_key_value_heads=8,
                head_dim=128, intermediate_size=25600, vocab_size=151936, tie_word_embeddings=False,
                rms_norm_eps=1e-6, rope_theta=1e6),
}


def tiny_config(layers=2, vocab=4096):
    """A small Qwen3 of the same structure, for quick parity tests."""
    return dict(hidden_size=512, num_hidden_layers=layers, num_attention_heads=8, num_key_value_heads=4,
                head_dim=64, intermediate_size=1024, vocab_size=vocab, tie_word_embeddings=True,
                rms_norm_eps=1e-6, rope_theta=1e6)


class _Arch:
    """Dimensions of a Qwen3 config, named as in the reference loader."""

    def _dims(self, c):
        self.cfg = dict(c, model_type="qwen3")
        self.D, self.L = c["hidden_size"], c["num_hidden_layers"]
        self.H, self.KV = c["num_attention_heads"], c["num_key_value_heads"]
        self.HD = c.get("head_dim", self.D // self.H)
        self.FF, self.eps, self.theta = c["intermediate_size"], c["rms_norm_eps"], c.get("rope_theta", 10000.0)
        self.V = c["vocab_size"]
        self.tied = c.get("tie_word_embeddings", False)

    def head_name(self):
        return "model.embed_tokens.weight" if self.tied else "lm_head.weight"

    def layer_params(self):
        """(N, K) of the fused layer matrices (formats/model.py:104-106)."""
        D, H, KV, HD, FF = self.D, self.H, self.KV, self.HD, self.FF
        return {"qkv": ((H + 2 * KV) * HD, D), "o": (D, H * HD), "gu": (2 * FF, D), "down": (D, FF)}

    def layer(self, i, device="cpu"):
        """Fused layer tensors: qkv = cat[q, k, v], gu = cat[gate, up] (formats/model.py:92-102)."""
        p = f"model.layers.{i}."
        a, m = p + "self_attn.", p + "mlp."
        t = lambda k: self.t(k, device)
        return {"qkv": torch.cat([t(a + "q_proj.weight"), t(a + "k_proj.weight"), t(a + "v_proj.weight")]),
                "o": t(a + "o_proj.weight"),
                "gu": torch.cat([t(m + "gate_proj.weight"), t(m + "up_proj.weight")]),
                "down": t(m + "down_proj.weight"),
                "ln1": t(p + "input_layernorm.weight"), "ln2": t(p + "post_attention_layernorm.weight"),
                "qn": t(a + "q_norm.weight"), "kn": t(a + "k_norm.weight")}

    def shapes(self):
        """name -> shape of every tensor of the checkpoint."""
        D, H, KV, HD, FF, V = self.D, self.H, self.KV, self.HD, self.FF, self.V
        s = {"model.embed_tokens.weight": (V, D), "model.norm.weight": (D,)}
        if not self.tied:
            s["lm_head.weight"] = (V, D)
        for i in range(self.L):
            p = f"model.layers.{i}."
            s.update({p + "self_attn.q_proj.weight": (H * HD, D), p + "self_attn.k_proj.weight": (KV * HD, D),
                      p + "self_attn.v_proj.weight": (KV * HD, D), p + "self_attn.o_proj.weight": (D, H * HD),
                      p + "self_attn.q_norm.weight": (HD,), p + "self_attn.k_norm.weight": (HD,),
                      p + "mlp.gate_proj.weight": (FF, D), p + "mlp.up_proj.weight": (FF, D),
                      p + "mlp.down_proj.weight": (D, FF), p + "input_layernorm.weight": (D,),
                      p + "post_attention_layernorm.weight": (D,)})
        return s


class RandomCkpt(_Arch):
    """Random-init Qwen3 made on demand: t(name) is the same bf16 tensor
    whenever it is asked for (the generator of each tensor is seeded by the
    model seed and the tensor name).  The values are drawn on `gen_device`
    (the GPU when there is one: a CPU generator needs minutes for an 8B
    model) and then moved to the device asked for, so every consumer of one
    RandomCkpt sees the same bits."""

    def __init__(self, cfg, seed=0, std=0.02, gen_device=None):
        self._dims(cfg)
        self.seed, self.std = seed, std
        self.gen_device = gen_device or ("cuda" if torch.cuda.is_available() else "cpu")
        self._shapes = self.shapes()
        self.eos = set()

    def t(self, name, device="cpu"):
        shape = self._shapes[name]
        if len(shape) == 1:
            return torch.ones(shape, dtype=torch.bfloat16, device=device)
        g = torch.Generator(device=self.gen_device)
        g.manual_seed((self.seed * 1000003 + zlib.crc32(name.encode())) % (2 ** 63))
        w = torch.randn(shape, generator=g, device=self.gen_device)
        return w.mul_(self.std).to(torch.bfloat16).to(device)


class Ckpt(_Arch):
    """A Hugging Face folder (config.json + *.safetensors) read one tensor at a
    time, with the reference loader's interface (formats/model.py:37-106)."""

    def __init__(self, path):
        from safetensors import safe_open
        self.dir = path
        cfg = json.load(open(os.path.join(path, "config.json")))
        if cfg.get("model_type") != "qwen3":
            raise NotImplementedError(f"model_type {cfg.get('model_type')} is not supported (qwen3)")
        self._dims(cfg)
        self.files = {}
        for f in sorted(os.listdir(path)):
            if f.endswith(".safetensors"):
                h = safe_open(os.path.join(path, f), framework="pt", device="cpu")
                for k in h.keys():
                    self.files[k] = h
        self.tied = cfg.get("tie_word_embeddings", False) or "lm_head.weight" not in self.files
        self.eos = set()

    def t(self, name, device="cpu"):
        return self.files[name].get_tensor(name).to(device)


def write_checkpoint(ck, path):
    """config.json + model.safetensors of a checkpoint object (small models)."""
    from safetensors.torch import save_file
    os.makedirs(path, exist_ok=True)
    json.dump(ck.cfg, open(os.path.join(path, "config.json"), "w"), indent=1)
    save_file({k: ck.t(k).contiguous() for k in ck.shapes()}, os.path.join(path, "model.safetensors"))
    return path
