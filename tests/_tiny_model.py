"""A random-init tiny Llama and a bijective character tokenizer (no downloads)."""

import torch


class CharTokenizer:
    """ids 0..93 <-> printable ASCII '!'..'~' (no spaces, so decode().strip() is lossless)."""

    eos_token_id = None
    pad_token_id = None

    def __init__(self, vocab: int = 94):
        self.vocab = vocab

    def encode(self, text: str, add_special_tokens: bool = True) -> list[int]:
        return [ord(c) - 33 for c in text]

    def decode(self, ids, skip_special_tokens: bool = True) -> str:
        return "".join(chr(33 + int(i)) for i in ids)

    def __call__(self, text: str, return_tensors: str = "pt"):
        ids = torch.tensor([self.encode(text)], dtype=torch.long)
        return {"input_ids": ids, "attention_mask": torch.ones_like(ids)}


def tiny_llama(device="cpu", dtype=torch.float32, layers: int = 2, heads: int = 8, kv_heads: int = 2, seed: int = 0,
               vocab: int = 94, hidden: int = 256):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=vocab, hidden_size=hidden, intermediate_size=512, num_hidden_layers=layers,
                      num_attention_heads=heads, num_key_value_heads=kv_heads, head_dim=128,
                      max_position_embeddings=4096, rope_theta=10000.0, attn_implementation="sdpa")
    model = LlamaForCausalLM(cfg).to(device=device, dtype=dtype).eval()
    model.generation_config.eos_token_id = None
    return model
