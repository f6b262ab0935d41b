"""GPU checks of the safetensors upload path: every tensor arrives in the
device arena bit for bit (tensors larger than one staging buffer, empty
tensors, every dtype), and a decoder built from an uploaded checkpoint with
the program's weight names decodes exactly like one built from the same
tensors in memory."""
import numpy as np
import pytest
import torch

from tests.helpers import from_f32, normal, rng

pytestmark = pytest.mark.gpu


def test_upload_roundtrip_bit_exact(tmp_path):
    from safetensors.torch import save_file
    from sandyrt_amd.weights import SafeTensors
    g = torch.Generator().manual_seed(0)
    tensors = {
        "big": torch.randn(5000, 4099, generator=g).to(torch.bfloat16),   # ~41 MB: spans staging buffers
        "f32": torch.randn(1023, 17, generator=g),
        "f16": torch.randn(33, generator=g).to(torch.float16),
        "i32": torch.randint(-2**31, 2**31 - 1, (77,), generator=g, dtype=torch.int32),
        "i64": torch.randint(-2**62, 2**62, (5, 3), generator=g, dtype=torch.int64),
        "u8": torch.randint(0, 255, (1001,), generator=g, dtype=torch.uint8),
        "empty": torch.zeros(0, 8),
    }
    p = str(tmp_path / "w.safetensors")
    save_file(tensors, p)
    st = SafeTensors(p)
    arena = st.upload()
    torch.cuda.synchronize()
    for name, t in tensors.items():
        got = st.get_tensor(name)
        assert got.shape == t.shape and got.dtype == t.dtype and got.is_cuda
        assert got.data_ptr() % 256 == 0 or t.numel() == 0
        assert torch.equal(got.cpu(), t), name
    assert st.get_tensor("absent") is None
    del arena
    st.close()


def test_decoder_from_checkpoint_matches_in_memory_weights(tmp_path):
    from safetensors.torch import save_file
    from sandyrt_amd.decode import DecodeConfig, TinyLlamaDecoder, random_weights, weights_from_safetensors
    from sandyrt_amd.device import HipDevice
    from sandyrt_amd.weights import SafeTensors
    cfg = DecodeConfig(layers=2, hidden=256, heads=8, kv_heads=2, head_dim=64, ffn=512, vocab=1000, max_context=128)
    w = random_weights(cfg, seed=5)
    hq, hk = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    ck = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["norm"], "lm_head.weight": w["lm_head"]}
    for i in range(cfg.layers):
        p = f"model.layers.{i}."
        qkv, gu = w[f"{i}.qkv"], w[f"{i}.gate_up"]
        ck.update({p + "input_layernorm.weight": w[f"{i}.in_norm"],
                   p + "post_attention_layernorm.weight": w[f"{i}.post_norm"],
                   p + "self_attn.q_proj.weight": qkv[:hq], p + "self_attn.k_proj.weight": qkv[hq:hq + hk],
                   p + "self_attn.v_proj.weight": qkv[hq + hk:], p + "self_attn.o_proj.weight": w[f"{i}.o"],
                   p + "mlp.gate_proj.weight": gu[:cfg.ffn], p + "mlp.up_proj.weight": gu[cfg.ffn:],
                   p + "mlp.down_proj.weight": w[f"{i}.down"]})
    path = str(tmp_path / "tinyllama-small.safetensors")
    save_file({k: v.cpu().contiguous() for k, v in ck.items()}, path)
    st = SafeTensors(path)
    st.upload()
    w2 = weights_from_safetensors(st, cfg)
    dev = HipDevice(0)
    try:
        a, b = TinyLlamaDecoder(dev, cfg, w), TinyLlamaDecoder(dev, cfg, w2)
        r = rng(6)
        ks = [from_f32(normal(r, (1, cfg.kv_heads, 20, cfg.head_dim)), torch.bfloat16) for _ in range(cfg.layers)]
        vs = [from_f32(normal(r, (1, cfg.kv_heads, 20, cfg.head_dim)), torch.bfloat16) for _ in range(cfg.layers)]
        for d in (a, b):
            d.prefill_cache(ks, vs)
            d.set_token(3)
        for _ in range(3):
            a.step()
            b.step()
            dev.synchronize()
            assert torch.equal(a.logits, b.logits)
    finally:
        dev.close()
        st.close()
