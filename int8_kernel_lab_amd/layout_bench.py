"""Throughput of the layout transforms (i8conv_nchw_to_nhwc & co.): 10
warmup + 100 back-to-back launches between two events on the null stream;
prints one JSON line per transform and tensor with GB/s of bytes read plus
bytes written.  The first five lines are the 51 MB headline tensors; the
rest are the activations and outputs of ResNet-50's stages at batch 64 (H x W
= 112 x 112 down to 7 x 7, where H x W is no multiple of 16 at 14 x 14 and
7 x 7).

    python -m int8_kernel_lab_amd.layout_bench
"""
import json

import torch

import int8_kernel_lab_amd as lab


def bw(name, fn, nbytes, args, out_bytes):
    src = torch.randint(-128, 127, (nbytes,), dtype=torch.int8, device="cuda")
    dst = torch.empty(out_bytes, dtype=torch.int8, device="cuda")
    for _ in range(10): fn(src.data_ptr(), dst.data_ptr(), *args)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(100): fn(src.data_ptr(), dst.data_ptr(), *args)
    e1.record(); torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 10
    print(json.dumps({"transform": name, "bytes_each_way": nbytes, "us": round(us, 2),
                      "gbps_read_plus_write": round(2 * nbytes / us / 1e3, 1)}), flush=True)
def main():
    n, h, w, c = 64, 56, 56, 256
    bw("nchw_to_nhwc 64x256x56x56 int8", lab.nchw_to_nhwc, n*c*h*w, (n, c, h, w), n*c*h*w)
    bw("nhwc_to_nchw 64x56x56x256 int8", lab.nhwc_to_nchw, n*c*h*w, (n, h, w, c), n*c*h*w)
    bw("pack_vect_c 64x56x56x256 v32", lab.pack_vect_c, n*c*h*w, (n, h, w, c, 32), n*c*h*w)
    bw("unpack_vect_c 64x56x56x256 v32", lab.unpack_vect_c, n*c*h*w, (n, h, w, c, 32), n*c*h*w)
    k = 256
    bw("nhwk_to_nkhw 16x56x56x256 int32", lab.nhwk_to_nkhw, 16*h*w*k*4, (16, h, w, k), 16*h*w*k*4)
    for (c, hw) in [(64, 112), (64, 56), (128, 28), (512, 28), (1024, 14), (2048, 7)]:
        e = n * c * hw * hw
        bw(f"nchw_to_nhwc 64x{c}x{hw}x{hw} int8", lab.nchw_to_nhwc, e, (n, c, hw, hw), e)
        bw(f"nhwc_to_nchw 64x{hw}x{hw}x{c} int8", lab.nhwc_to_nchw, e, (n, hw, hw, c), e)
    for (k, hw) in [(512, 28), (1024, 14), (2048, 7)]:
        e = n * k * hw * hw * 4
        bw(f"nhwk_to_nkhw 64x{hw}x{hw}x{k} int32", lab.nhwk_to_nkhw, e, (n, hw, hw, k), e)


if __name__ == "__main__":
    main()
