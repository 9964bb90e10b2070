"""Write the golden vectors in tests/golden/ by running the reference's CPU path.

Run once, in the build container (the reference is not present on the GPU
box), from the repository root:

    PYTHONHASHSEED=0 python tests/golden/gen_fixtures.py /root/reference

The reference module patches torch globally when imported, so this script
runs it in a child process of its own.  It records inputs and outputs only
(numpy arrays, no pickles) into ``tests/golden/fixtures.npz`` plus a JSON
index ``tests/golden/fixtures.json``.  Inputs come from seeded CPU
generators; the seeds are listed in the JSON index.

Vectors written (all through the reference's public entry points):
  * ``mx_tensor.quantize`` packed bytes/words and scales, and
    ``.dequantize()`` output, for int8d/int4d/int2d/int1d/int3d, float4d,
    float8d, int8dv, int4dv, int4dh, over seeded, ragged, tie, zero,
    sign-of-zero, tiny and outlier inputs, block sizes 16..256 and fp16/bf16
    inputs;
  * ``qa @ qb`` (``_dispatch_qgemm``) packed output, scales and dtype for
    int8d/int4d/int2d/int1d/float4d/float8d operands, K a multiple of the
    block and not;
  * ``_QGemmSTE.apply`` forward output;
  * ``mx_linear.from_linear(...)(x)`` with and without bias;
  * ``kv_cache_quantizer`` append/get with asymmetric V;
  * the int4dh hash seed under PYTHONHASHSEED=0;
  * quantize of blocks holding NaN and infinities (NaN / infinite scales).
"""
from __future__ import annotations

import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def _child(ref_dir: str) -> None:
    import numpy as np
    import torch

    torch.set_num_threads(1)
    sys.path.insert(0, ref_dir)
    import mxtorch as mx  # noqa: E402  (the reference, read-only)

    arrays = {}
    index = {"cases": [], "hash_seed": {}}

    def put(key, t):
        if isinstance(t, torch.Tensor):
            t = t.detach().cpu()
            if t.dtype == torch.bfloat16:
                t = t.view(torch.int16)
            arrays[key] = t.numpy()
        else:
            arrays[key] = np.asarray(t)

    def gen(seed):
        g = torch.Generator()
        g.manual_seed(seed)
        return g

    # ---------------- quantize / dequantize ----------------
    inputs = {}
    inputs["randn_4x256"] = (torch.randn(4, 256, generator=gen(101)), 101)
    inputs["randn_ragged_300"] = (torch.randn(300, generator=gen(102)), 102)
    inputs["randn_2x3x50"] = (torch.randn(2, 3, 50, generator=gen(103)), 103)
    x = torch.randn(2048, generator=gen(104))
    mask = torch.rand(2048, generator=gen(105)) < 0.01
    x[mask] *= 50
    inputs["outliers_2048"] = (x, 104)
    z = torch.zeros(384)
    z[128:256] = -0.0
    z[300] = 1e-30
    z[301] = -1e-40
    inputs["zeros_signed_384"] = (z, 0)
    tiny = torch.randn(256, generator=gen(106)) * 1e-38
    inputs["tiny_256"] = (tiny, 106)
    const = torch.full((256,), 0.3)
    const[128:] = -2.5
    inputs["const_256"] = (const, 0)
    # ties for the float grids: values placed exactly on the bucket mids
    for bits in (4, 8):
        g = mx._get_minifloat_grid(bits)
        mids = (g[:-1] + g[1:]) * 0.5
        t = torch.cat([mids, torch.tensor([1.0]), torch.nextafter(mids, torch.full_like(mids, 2.0)),
                       torch.nextafter(mids, torch.full_like(mids, -2.0)), g])
        inputs[f"grid_ties_f{bits}"] = (t, 0)
    # ties for the int quantizer: k + 0.5 steps of a block whose absmax is 127
    it = torch.arange(-127.0, 127.5, 0.5)
    it = it[torch.randperm(it.numel(), generator=gen(107))][:256]
    it[0] = 127.0
    inputs["int_ties_256"] = (it, 107)
    inputs["randn_fp16_3x128"] = (torch.randn(3, 128, generator=gen(108)).half(), 108)
    inputs["randn_bf16_3x128"] = (torch.randn(3, 128, generator=gen(109)).bfloat16(), 109)

    dtypes = ["int8d", "int4d", "int2d", "int1d", "int3d", "float4d", "float8d",
              "int8dv", "int4dv", "int4u"]
    blocks = {"randn_4x256": (16, 32, 64, 128, 256), "randn_ragged_300": (128, 64),
              "randn_2x3x50": (128, 32)}
    for iname, (xin, seed) in inputs.items():
        for dname in dtypes:
            for block in blocks.get(iname, (128,)):
                dt = mx.get_mx_dtype(dname)
                q = mx.mx_tensor.quantize(xin, dt, block)
                key = f"q/{iname}/{dname}/{block}"
                put(key + "/packed", q._mx_packed)
                put(key + "/scales", q._mx_scales)
                put(key + "/dequant", q.dequantize())
                index["cases"].append({"kind": "quantize", "key": key, "input": iname,
                                       "dtype": dname, "block": block, "n": int(q._mx_n),
                                       "shape": list(xin.shape), "seed": seed,
                                       "packed_dtype": str(q._mx_packed.dtype)})
        put(f"in/{iname}", xin)
        index["cases"].append({"kind": "input", "key": f"in/{iname}", "dtype": str(xin.dtype),
                               "shape": list(xin.shape), "seed": seed})

    # non-finite blocks: torch's amax propagates NaN, so a block holding a
    # NaN gets a NaN scale; an infinity gives an infinite scale (its codes
    # come from NaN and zero quotients)
    nf = torch.randn(5, 128, generator=gen(140))
    nf[1, 2] = float("nan")
    nf[2, 44] = float("inf")
    nf[3, 16] = float("nan")
    nf[3, 17] = float("-inf")
    nf[4, 100] = float("-inf")
    put("in/nonfinite_5x128", nf)
    for dname in ("int8d", "int4d", "int2d", "int1d", "float4d", "float8d", "int8dv", "int4dh"):
        dt = mx.get_mx_dtype(dname)
        q = mx.mx_tensor.quantize(nf, dt, 128)
        key = f"qnf/nonfinite_5x128/{dname}/128"
        put(key + "/packed", q._mx_packed)
        put(key + "/scales", q._mx_scales)
        put(key + "/dequant", q.dequantize())
        index["cases"].append({"kind": "quantize_nonfinite", "key": key, "input": "nonfinite_5x128",
                               "dtype": dname, "block": 128, "n": int(q._mx_n), "shape": [5, 128],
                               "seed": 140, "packed_dtype": str(q._mx_packed.dtype)})

    # int4dh: the seed is hash(name) % 2**31, fixed here by PYTHONHASHSEED
    index["hash_seed"]["int4dh"] = hash("int4dh") % (2 ** 31)
    index["hash_seed"]["float4dh"] = hash("float4dh") % (2 ** 31)
    index["hash_seed"]["PYTHONHASHSEED"] = os.environ.get("PYTHONHASHSEED")
    had_inputs = {"h_8x128": torch.randn(8, 128, generator=gen(110)),
                  "h_4x100": torch.randn(4, 100, generator=gen(111)),
                  "h_1d_512": torch.randn(512, generator=gen(112)),
                  "h_1d_300": torch.randn(300, generator=gen(113))}
    for iname, xin in had_inputs.items():
        put(f"in/{iname}", xin)
        for dname in ("int4dh", "int8dh", "float4dh"):
            dt = mx.get_mx_dtype(dname)
            q = mx.mx_tensor.quantize(xin, dt, 128)
            key = f"q/{iname}/{dname}/128"
            put(key + "/packed", q._mx_packed)
            put(key + "/scales", q._mx_scales)
            put(key + "/dequant", q.dequantize())
            index["cases"].append({"kind": "quantize", "key": key, "input": iname,
                                   "dtype": dname, "block": 128, "n": int(q._mx_n),
                                   "shape": list(xin.shape), "seed": None,
                                   "packed_dtype": str(q._mx_packed.dtype)})
    index["hash_seed"]["int8dh"] = hash("int8dh") % (2 ** 31)
    signs = mx.hadamard_rotation(128, seed=index["hash_seed"]["int4dh"]).signs
    put("signs/int4dh/128", signs)

    # ---------------- qa @ qb ----------------
    gemm_cases = [("int8d", 32, 256, 64, 120), ("int4d", 32, 256, 64, 121),
                  ("int8d", 16, 100, 24, 122), ("int2d", 16, 128, 32, 123),
                  ("int1d", 16, 128, 32, 124), ("float4d", 16, 128, 32, 125),
                  ("float8d", 16, 128, 32, 126), ("int8d", 24, 384, 136, 127),
                  ("int4d", 24, 200, 72, 128)]
    for dname, M, K, N, seed in gemm_cases:
        g = gen(seed)
        A = torch.randn(M, K, generator=g)
        B = torch.randn(K, N, generator=g)
        dt = mx.get_mx_dtype(dname)
        qa = mx.mx_tensor.quantize(A, dt, 128)
        qb = mx.mx_tensor.quantize(B, dt, 128)
        qc = qa @ qb
        key = f"mm/{dname}/{M}x{K}x{N}"
        put(key + "/A", A)
        put(key + "/B", B)
        put(key + "/packed", qc._mx_packed)
        put(key + "/scales", qc._mx_scales)
        put(key + "/dequant", qc.dequantize())
        ste = mx._QGemmSTE.apply(A, B, dt, 128)
        put(key + "/ste", ste)
        index["cases"].append({"kind": "matmul", "key": key, "dtype": dname, "M": M, "K": K,
                               "N": N, "seed": seed, "out_dtype": qc._mx_dtype.name,
                               "out_block": int(qc._mx_block),
                               "packed_dtype": str(qc._mx_packed.dtype),
                               "result_type": type(qc).__name__})

    # ---------------- mx_linear ----------------
    for dname, bias, seed in (("int4d", False, 130), ("int4d", True, 131), ("int8d", True, 132)):
        g = gen(seed)
        lin = torch.nn.Linear(128, 192, bias=bias)
        with torch.no_grad():
            lin.weight.copy_(torch.randn(192, 128, generator=g) * 0.02)
            if bias:
                lin.bias.copy_(torch.randn(192, generator=g))
        x = torch.randn(4, 128, generator=g)
        m = mx.mx_linear.from_linear(lin, mx.get_mx_dtype(dname), 128)
        y = m(x)
        key = f"lin/{dname}/bias{int(bias)}"
        put(key + "/W", lin.weight.data)
        if bias:
            put(key + "/bias", lin.bias.data)
        put(key + "/x", x)
        put(key + "/y", y)
        put(key + "/w_packed", m._mx_weight._mx_packed)
        put(key + "/w_scales", m._mx_weight._mx_scales)
        index["cases"].append({"kind": "linear", "key": key, "dtype": dname, "bias": bias,
                               "in": 128, "out": 192, "seed": seed})

    # ---------------- kv cache ----------------
    for dname, seed in (("int8d", 140), ("int4d", 141), ("int8dv", 142)):
        g = gen(seed)
        cache = mx.kv_cache_quantizer(n_heads=4, head_dim=128, dtype=dname)
        ks, vs = [], []
        for _ in range(3):
            k = torch.randn(2, 4, 1, 128, generator=g)
            v = torch.randn(2, 4, 1, 128, generator=g) + 0.5
            cache.append_kv(k, v)
            ks.append(k)
            vs.append(v)
        K_all, V_all = cache.get()
        key = f"kv/{dname}"
        put(key + "/k", torch.stack(ks))
        put(key + "/v", torch.stack(vs))
        put(key + "/K", K_all)
        put(key + "/V", V_all)
        kq, vq = cache.get_quantized()
        for t in range(3):
            put(f"{key}/kq{t}/packed", kq[t]._mx_packed)
            put(f"{key}/kq{t}/scales", kq[t]._mx_scales)
            put(f"{key}/vq{t}/packed", vq[t]._mx_packed)
            put(f"{key}/vq{t}/scales", vq[t]._mx_scales)
        index["cases"].append({"kind": "kv", "key": key, "dtype": dname, "seed": seed,
                               "B": 2, "H": 4, "D": 128, "T": 3})

    # ---------------- quantized element-wise ops (mxtorch.py:5321-5497, 6177-6193) ----------------
    for dname, seed in (("int8d", 150), ("int4d", 151), ("int2d", 152)):
        g = gen(seed)
        A = torch.randn(4, 256, generator=g)
        B = torch.randn(4, 256, generator=g)
        dt = mx.get_mx_dtype(dname)
        qa_ = mx.mx_tensor.quantize(A, dt, 128)
        qb_ = mx.mx_tensor.quantize(B, dt, 128)
        qw_ = mx.mx_tensor.quantize(B * 37.0, dt, 128)  # block scales more than 2:1 apart
        key = f"ew/{dname}"
        put(key + "/A", A)
        put(key + "/B", B)
        ops = {"add": qa_ + qb_, "sub": qa_ - qb_, "mul": qa_ * qb_, "neg": -qa_,
               "addw": qa_ + qw_, "subw": qa_ - qw_, "mulw": qa_ * qw_}
        out_names = {}
        for opname, res in ops.items():
            put(f"{key}/{opname}/packed", res._mx_packed)
            put(f"{key}/{opname}/scales", res._mx_scales)
            put(f"{key}/{opname}/dequant", res.dequantize())
            out_names[opname] = res._mx_dtype.name
        index["cases"].append({"kind": "elementwise", "key": key, "dtype": dname, "seed": seed,
                               "shape": [4, 256], "wide_factor": 37.0, "out_dtype": out_names})

    # ---------------- to_mx on a small model, and save_quantized (mxtorch.py:9744-9898) ----------------
    class _MLP(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.fc1 = torch.nn.Linear(64, 128)
            self.act = torch.nn.ReLU()
            self.norm = torch.nn.LayerNorm(128)
            self.fc2 = torch.nn.Linear(128, 32)

        def forward(self, x):
            return self.fc2(self.norm(self.act(self.fc1(x))))

    g = gen(160)
    model = _MLP()
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.1 + (1.0 if p.ndim == 1 and p.numel() == 128 else 0.0))
    x = torch.randn(6, 64, generator=g)
    for name, p in model.named_parameters():
        put(f"tomx/param/{name}", p.data)
    put("tomx/x", x)
    mx.to_mx(model, "int4d")
    y = model(x)
    put("tomx/y", y.dequantize() if isinstance(y, mx.mx_tensor) else y)
    for attr in ("fc1", "fc2"):
        lin = getattr(model, attr)
        put(f"tomx/{attr}/w_packed", lin._mx_weight._mx_packed)
        put(f"tomx/{attr}/w_scales", lin._mx_weight._mx_scales)
    norm_w = model.norm.weight.data
    norm_b = model.norm.bias.data
    put("tomx/norm/w_packed", norm_w._mx_packed)
    put("tomx/norm/w_scales", norm_w._mx_scales)
    put("tomx/norm/b_packed", norm_b._mx_packed)
    put("tomx/norm/b_scales", norm_b._mx_scales)
    ckpt_path = os.path.join(HERE, "ref_checkpoint.pt")
    mx.save_quantized(model, ckpt_path)
    index["cases"].append({"kind": "to_mx", "key": "tomx", "dtype": "int4d", "seed": 160,
                           "modules": {n: type(mm).__name__ for n, mm in model.named_children()},
                           "checkpoint": os.path.basename(ckpt_path)})

    # ---------------- mx_multihead_attention (mxtorch.py:7800-7877) ----------------
    g = gen(170)
    mha = torch.nn.MultiheadAttention(128, 4, batch_first=True)
    with torch.no_grad():
        for p in mha.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.05)
    q = torch.randn(2, 8, 128, generator=g)
    for name, p in mha.named_parameters():
        put(f"mha/param/{name}", p.data)
    m = mx.mx_multihead_attention.from_mha(mha, mx.get_mx_dtype("int8d"), 128)
    out, attn = m(q, q, q)
    put("mha/q", q)
    put("mha/in_proj/packed", m.in_proj_weight._mx_packed)
    put("mha/in_proj/scales", m.in_proj_weight._mx_scales)
    put("mha/out_proj/packed", m.out_proj._mx_weight._mx_packed)
    put("mha/out_proj/scales", m.out_proj._mx_weight._mx_scales)
    put("mha/out/packed", out._mx_packed)
    put("mha/out/scales", out._mx_scales)
    put("mha/out/dequant", out.dequantize())
    put("mha/attn", attn)
    index["cases"].append({"kind": "mha", "key": "mha", "dtype": "int8d", "seed": 170, "embed": 128,
                           "heads": 4, "shape": [2, 8, 128], "out_dtype": out._mx_dtype.name})

    # ---------------- mx_transformer_encoder_layer (mxtorch.py:9161-9260) ----------------
    g = gen(180)
    enc = torch.nn.TransformerEncoderLayer(d_model=128, nhead=4, dim_feedforward=256, dropout=0.0,
                                           batch_first=True)
    with torch.no_grad():
        for name, p in enc.named_parameters():
            base = 1.0 if ("norm" in name and name.endswith("weight")) else 0.0
            p.copy_(torch.randn(p.shape, generator=g) * 0.05 + base)
    enc.eval()
    src = torch.randn(2, 8, 128, generator=g)
    for name, p in enc.named_parameters():
        put(f"enc/param/{name}", p.data)
    m = mx.mx_transformer_encoder_layer.from_encoder_layer(enc, mx.get_mx_dtype("int8d"), 128)
    m.eval()
    y = m(src)
    put("enc/src", src)
    put("enc/y", y.dequantize() if isinstance(y, mx.mx_tensor) else y)
    put("enc/linear1/w_packed", m.linear1._mx_weight._mx_packed)
    put("enc/linear2/w_packed", m.linear2._mx_weight._mx_packed)
    index["cases"].append({"kind": "encoder_layer", "key": "enc", "dtype": "int8d", "seed": 180, "d_model": 128,
                           "nhead": 4, "ff": 256, "shape": [2, 8, 128]})

    # ---------------- vector_quantize (mxtorch.py:2946-2994) ----------------
    g = gen(190)
    xv = torch.randn(16, 300, generator=g)
    xv[torch.rand(16, 300, generator=g) < 0.01] *= 40
    xv[3] = 0.0                      # an all-zero row
    xv[5, ::7] = torch.arange(43, dtype=torch.float32) * 0.5 - 10.5   # exact halves of a step after scaling
    put("vq/x", xv)
    for dname, axis in (("int8d", 1), ("int8d", 0), ("int4d", 1), ("int2d", 0), ("int16d", 1)):
        codes, scales = mx.vector_quantize(xv, dname, axis=axis)
        key = f"vq/{dname}/axis{axis}"
        put(key + "/codes", codes)
        put(key + "/scales", scales)
        put(key + "/dequant", mx.vector_dequantize(codes, scales, axis=axis))
        index["cases"].append({"kind": "vector_quantize", "key": key, "dtype": dname, "axis": axis, "seed": 190,
                               "shape": [16, 300]})

    # ---------------- pack KATs (mxtorch_test.py:86-112) ----------------
    vals = torch.tensor([3, -2, 7, -8, 0, 1, -1, 4], dtype=torch.int8)
    put("kat/pack4", mx.bit_packer.pack(vals, 4))
    put("kat/pack1", mx.bit_packer.pack(torch.tensor([0, 1, 0, 1, 1, 0, 1, 0], dtype=torch.int8), 1))
    put("kat/pack2", mx.bit_packer.pack(torch.tensor([1, -2, 0, -1, 1, -2, 0, 1], dtype=torch.int8), 2))
    put("kat/pack3", mx.bit_packer.pack_arb(torch.tensor([3, -4, 2, -3, 0, 1, -1, 3], dtype=torch.int32), 3))
    put("kat/pack16", mx.bit_packer.pack_arb(torch.tensor([32767, -32767, 5, -1, 0], dtype=torch.int32), 16))
    put("grid/4", mx._get_minifloat_grid(4))
    put("grid/8", mx._get_minifloat_grid(8))

    np.savez_compressed(os.path.join(HERE, "fixtures.npz"), **arrays)
    with open(os.path.join(HERE, "fixtures.json"), "w") as f:
        json.dump(index, f, indent=1, sort_keys=True)
    print(f"wrote {len(arrays)} arrays, {len(index['cases'])} cases")


def main() -> None:
    if len(sys.argv) >= 3 and sys.argv[1] == "--child":
        _child(sys.argv[2])
        return
    ref_dir = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    env = dict(os.environ, PYTHONHASHSEED="0")
    subprocess.run([sys.executable, os.path.abspath(__file__), "--child", ref_dir],
                   env=env, check=True)


if __name__ == "__main__":
    main()
