"""Timing of tgohip_linear at the Qwen3-8B projection shapes.

    python -m tgo_amd.linear_bench [--rows 1,8,64] [--form 3] [--x f16|f32|x2]
                                   [--shapes qkv,o,gateup,down,lmhead,c3a,c3b,c3c]

Each shape's weight is synthesized in enough copies (over 800 MB in all) that
back-to-back launches cycle through them and none stays in the 256 MB
last-level cache: the weight stream comes from HBM, as it does in a model
step. Per launch: the median of five timings of 4 passes over the copies
(HIP events on the launch stream). Reported per launch: the algorithmic bytes
(weights + scales once, activations in, output out) and their rate against
MI355X's 8 TB/s, the algorithmic flops 2*M*K*N and their rate against the dense
f16 MFMA peak of 2.5 PFLOP/s, and the roofline fraction max(bytes/8 TB/s,
flops/2.5 PFLOP/s) / time. Activations N(0,1): f16 (--x f16), f32 (f32), or
the f16 hi/lo pair of tgo's arithmetic (x2, TGOHIP_F16X2); the output f16.
The c3* shapes are BASELINE config 3's [K x N]: [4096 x 12288], [12288 x 4096],
[4096 x 6144].
"""
import argparse

import torch

import tgo_amd

SHAPES = [("qkv", 4096, 6144), ("o", 4096, 4096), ("gateup", 4096, 24576),
          ("down", 12288, 4096), ("lmhead", 4096, 151936),
          ("c3a", 4096, 12288), ("c3b", 12288, 4096), ("c3c", 4096, 6144)]
PEAK_GBPS = 8000.0
PEAK_TFLOPS = 2500.0


def weight_bytes(form, K, N):
    per = {tgo_amd.FORM_I4_SYM: 0.5 + 2 / 32, tgo_amd.FORM_I4_TGO: 0.5 + 4 / 128,
           tgo_amd.FORM_I8: 1 + 2 / 32, tgo_amd.FORM_F16: 2}[form]
    return K * N * per


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--rows", default="1,8")
    p.add_argument("--form", type=int, default=tgo_amd.FORM_I4_SYM)
    p.add_argument("--x", default="f16", choices=["f16", "f32", "x2"])
    p.add_argument("--shapes", default=",".join(s[0] for s in SHAPES[:5]))
    args = p.parse_args()
    rows = [int(r) for r in args.rows.split(",")]
    want = set(args.shapes.split(","))
    xdt = {"f16": tgo_amd.F16, "f32": tgo_amd.F32, "x2": tgo_amd.F16X2}[args.x]
    xbytes = 2 if args.x == "f16" else 4
    ctx = tgo_amd.Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    print("%-7s %5s %6s %7s %6s %10s %9s %7s %9s %7s %8s" % (
        "shape", "M", "K", "N", "copies", "us/launch", "GB/s", "of_8TB", "TFLOP/s", "of_2.5P",
        "roofline"))
    for name, K, N in SHAPES:
        if name not in want:
            continue
        wb = weight_bytes(args.form, K, N)
        copies = max(2, min(64, int(800e6 // wb) + 1))
        hs = [ctx.weight_synth(args.form, K, N, 7 + i, 1, 0.02) for i in range(copies)]
        try:
            for M in rows:
                if args.x == "f16":
                    x = torch.randn(M, K, device="cuda").half()
                elif args.x == "f32":
                    x = torch.randn(M, K, device="cuda")
                else:
                    xf = torch.randn(M, K, device="cuda")
                    hi = xf.half()
                    lo = (xf - hi.float()).half()
                    x = torch.cat([hi.reshape(-1), lo.reshape(-1)])
                y = torch.empty(M, N, device="cuda", dtype=torch.float16)
                for h in hs:
                    ctx.linear(h, x, M, y, x_dtype=xdt, y_dtype=tgo_amd.F16)
                torch.cuda.synchronize()
                times = []
                for _ in range(5):
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(4):
                        for h in hs:
                            ctx.linear(h, x, M, y, x_dtype=xdt, y_dtype=tgo_amd.F16)
                    e1.record()
                    torch.cuda.synchronize()
                    times.append(e0.elapsed_time(e1) / (4 * copies))
                ms = sorted(times)[2]
                by = wb + M * K * xbytes + M * N * 2
                fl = 2.0 * M * K * N
                gbps = by / ms / 1e6
                tfs = fl / ms / 1e9
                roof = max(by / (PEAK_GBPS * 1e6), fl / (PEAK_TFLOPS * 1e9)) / ms
                print("%-7s %5d %6d %7d %6d %10.2f %9.0f %7.3f %9.1f %7.3f %8.3f" % (
                    name, M, K, N, copies, ms * 1e3, gbps, gbps / PEAK_GBPS, tfs,
                    tfs / PEAK_TFLOPS, roof), flush=True)
        finally:
            for h in hs:
                ctx.weight_free(h)
    ctx.close()


if __name__ == "__main__":
    main()
