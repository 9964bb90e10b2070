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
  * the int4dh hash seed under PYTHONHASHSEED=0.
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
