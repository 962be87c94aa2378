"""Timing of tgohip_linear at the Qwen3-8B projection shapes.

    python -m tgo_amd.linear_bench [--rows 1,8,64] [--form 3] [--shapes qkv,o,gateup,down,lmhead]

Each shape's weight is synthesized in enough copies (over 800 MB in all) that
back-to-back launches cycle through them and none stays in the 256 MB
last-level cache: the weight stream comes from HBM, as it does in a model
step. Per launch: the median of five timings of 4 passes over the copies
(HIP events on the launch stream), the weight bytes it streams and their rate
against MI355X's 8 TB/s. Activations are f16 N(0,1), the output f16.
"""
import argparse

import torch

import tgo_amd

SHAPES = [("qkv", 4096, 6144), ("o", 4096, 4096), ("gateup", 4096, 24576),
          ("down", 12288, 4096), ("lmhead", 4096, 151936)]
PEAK_GBPS = 8000.0


def weight_bytes(form, K, N):
    per = {tgo_amd.FORM_I4_SYM: 0.5 + 2 / 32, tgo_amd.FORM_I4_TGO: 0.5 + 4 / 128,
           tgo_amd.FORM_I8: 1 + 2 / 32, tgo_amd.FORM_F16: 2}[form]
    return K * N * per


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--rows", default="1,8")
    p.add_argument("--form", type=int, default=tgo_amd.FORM_I4_SYM)
    p.add_argument("--shapes", default=",".join(s[0] for s in SHAPES))
    args = p.parse_args()
    rows = [int(r) for r in args.rows.split(",")]
    want = set(args.shapes.split(","))
    ctx = tgo_amd.Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    print("%-7s %5s %6s %7s %6s %10s %10s %7s" % ("shape", "M", "K", "N", "copies", "us/launch",
                                                 "GB/s", "of_8TB"))
    for name, K, N in SHAPES:
        if name not in want:
            continue
        wb = weight_bytes(args.form, K, N)
        copies = max(2, min(64, int(800e6 // wb) + 1))
        hs = [ctx.weight_synth(args.form, K, N, 7 + i, 1, 0.02) for i in range(copies)]
        try:
            for M in rows:
                x = torch.randn(M, K, device="cuda").half()
                y = torch.empty(M, N, device="cuda", dtype=torch.float16)
                for h in hs:
                    ctx.linear(h, x, M, y, x_dtype=tgo_amd.F16, y_dtype=tgo_amd.F16)
                torch.cuda.synchronize()
                times = []
                for _ in range(5):
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(4):
                        for h in hs:
                            ctx.linear(h, x, M, y, x_dtype=tgo_amd.F16, y_dtype=tgo_amd.F16)
                    e1.record()
                    torch.cuda.synchronize()
                    times.append(e0.elapsed_time(e1) / (4 * copies))
                ms = sorted(times)[2]
                gbps = wb / ms / 1e6
                print("%-7s %5d %6d %7d %6d %10.2f %10.0f %7.3f" % (name, M, K, N, copies, ms * 1e3,
                                                                   gbps, gbps / PEAK_GBPS),
                      flush=True)
        finally:
            for h in hs:
                ctx.weight_free(h)
    ctx.close()


if __name__ == "__main__":
    main()
