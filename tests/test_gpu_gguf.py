"""GGUF ingestion on the GPU: a synthetic checkpoint (every kernel type, a BF16 LM head, a
fused Q4_K expert stack with its Q4_K router and shared expert) is written with the GGUF
writer, uploaded through the pinned staging path, and fed unchanged to the kernels; every
result is compared bit-exactly with the oracle run on the bytes read back from the file."""
import numpy as np
import pytest
import torch

from aipu_amd import device as dev
from aipu_amd import gguf
from oracle import c_oracle as co
from oracle import glm_oracle as go
from oracle import q4k_oracle as qo

from .gpu_util import assert_bits_equal, d_bf16, h_bits, note

pytestmark = pytest.mark.gpu

E, H, I, TOPK = 8, 512, 256, 2


def _checkpoint(path, rng):
    t = [
        ("blk.0.ffn_down.weight", gguf.GGML_Q4_K, [1024, 96], qo.random_q4k_blocks(rng, 384)),
        ("blk.0.attn_output.weight", gguf.GGML_Q6_K, [512, 40], qo.random_q6k_blocks(rng, 80)),
        ("blk.0.attn_q.weight", gguf.GGML_Q8_0, [512, 40], qo.random_q8_0_blocks(rng, 640)),
        ("blk.0.attn_kv.weight", gguf.GGML_F16, [512, 40], qo.random_f16_weights(rng, 512 * 40).view(np.uint8)),
        ("output.weight", gguf.GGML_BF16, [256, 300], qo.random_bf16(rng, (300, 256)).view(np.uint8)),
        ("output_norm.weight", gguf.GGML_F32, [256], rng.standard_normal(256).astype(np.float32).view(np.uint8)),
        ("blk.1.ffn_gate_inp.weight", gguf.GGML_Q4_K, [H, E], qo.random_q4k_blocks(rng, E * H // 256)),
        ("blk.1.ffn_gate_exps.weight", gguf.GGML_Q4_K, [H, I, E], qo.random_q4k_blocks(rng, E * I * H // 256)),
        ("blk.1.ffn_up_exps.weight", gguf.GGML_Q4_K, [H, I, E], qo.random_q4k_blocks(rng, E * I * H // 256)),
        ("blk.1.ffn_down_exps.weight", gguf.GGML_Q4_K, [I, H, E], qo.random_q4k_blocks(rng, E * H * I // 256)),
        ("blk.1.ffn_gate_shexp.weight", gguf.GGML_Q4_K, [H, I], qo.random_q4k_blocks(rng, I * H // 256)),
        ("blk.1.ffn_up_shexp.weight", gguf.GGML_Q4_K, [H, I], qo.random_q4k_blocks(rng, I * H // 256)),
        ("blk.1.ffn_down_shexp.weight", gguf.GGML_Q4_K, [I, H], qo.random_q4k_blocks(rng, H * I // 256)),
    ]
    path.write_bytes(gguf.write_gguf([(n, ty, d, np.ascontiguousarray(r).tobytes()) for n, ty, d, r in t]))
    return t


def test_gguf_upload_and_run(tmp_path):
    note("gguf upload + kernels")
    rng = np.random.default_rng(21)
    p = tmp_path / "ckpt.gguf"
    _checkpoint(p, rng)
    f = gguf.GGUFFile(str(p))
    dts = f.upload_all("cuda", staging_bytes=4096)      # many staging rounds per tensor
    torch.cuda.synchronize()
    for t in f.tensors:
        host = np.asarray(f.host_bytes(t.name))
        assert np.array_equal(dts[t.name].data.cpu().numpy(), host), t.name

    # 2-D weights of every kernel type, reference order (bit-exact)
    x_bits = qo.random_bf16(rng, (2, 1024))
    for name in ("blk.0.ffn_down.weight", "blk.0.attn_output.weight", "blk.0.attn_q.weight", "blk.0.attn_kv.weight"):
        d = dts[name]
        xb = np.ascontiguousarray(x_bits[:, :d.K])
        y = dev.gemv(d.ggml_type, d.data, d.N, d.K, d_bf16(xb), mode="ref")
        _, ye = co.gemv_ref(d.ggml_type, np.asarray(f.host_bytes(name)), d.N, d.K, xb)
        assert_bits_equal(h_bits(y), ye, name)

    # LM head straight from the BF16 tensor
    lm = dts["output.weight"]
    xl = qo.random_bf16(rng, lm.K)
    lg, am = dev.lm_head(lm.as_bf16_rows(), d_bf16(xl))
    le, ae = co.lm_head(np.asarray(f.host_bytes("output.weight")).view(np.uint16).reshape(lm.N, lm.K), xl)
    assert_bits_equal(h_bits(lg), le, "lm head from gguf")
    assert int(am.cpu()[0]) == ae

    # MoE decode step on the fused expert stacks (reference mode, bit-exact)
    g, u, dn = (dts[f"blk.1.ffn_{k}_exps.weight"] for k in ("gate", "up", "down"))
    assert (g.K, g.N, g.E) == (H, I, E) and (dn.K, dn.N, dn.E) == (I, H, E)
    assert g.expert(3).numel() == I * H // 256 * 144
    rw = dts["blk.1.ffn_gate_inp.weight"]
    sh = tuple(dts[f"blk.1.ffn_{k}_shexp.weight"].data for k in ("gate", "up", "down"))
    xm = qo.random_bf16(rng, H, scale=0.05)
    y, sel, sw = dev.moe_swiglu_decode(gguf.GGML_Q4_K, rw.data, gguf.GGML_Q4_K, g.data, u.data, dn.data, E, H, I,
                                       TOPK, d_bf16(xm), mode="ref", shared=sh)
    hb = {t.name: np.asarray(f.host_bytes(t.name)) for t in f.tensors}
    r = go.moe_decode_ref(xm, gguf.GGML_Q4_K, hb["blk.1.ffn_gate_inp.weight"],
                          (hb["blk.1.ffn_gate_exps.weight"], hb["blk.1.ffn_up_exps.weight"],
                           hb["blk.1.ffn_down_exps.weight"]), gguf.GGML_Q4_K, E, H, I, TOPK,
                          shared=(hb["blk.1.ffn_gate_shexp.weight"], hb["blk.1.ffn_up_shexp.weight"],
                                  hb["blk.1.ffn_down_shexp.weight"]))
    assert np.array_equal(sel.cpu().numpy(), r["sel_idx"])
    assert_bits_equal(h_bits(sw), r["sel_w"], "moe sel_w")
    assert_bits_equal(h_bits(y), r["y"], "moe y from gguf")


def test_gguf_upload_kind_filter(tmp_path):
    note("gguf kind filter")
    rng = np.random.default_rng(22)
    p = tmp_path / "ckpt.gguf"
    _checkpoint(p, rng)
    f = gguf.GGUFFile(str(p))
    hot = f.upload_all("cuda", kind="resident_hot")
    exp = f.upload_all("cuda", kind="streamed_expert")
    assert set(exp) == {"blk.1.ffn_gate_exps.weight", "blk.1.ffn_up_exps.weight", "blk.1.ffn_down_exps.weight"}
    assert not set(hot) & set(exp) and len(hot) + len(exp) == len(f.tensors)
