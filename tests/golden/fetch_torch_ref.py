"""Copy the GEMM golden vectors that the reference repository holds as data.

Source: <reference>/benchmarks/torch_ref/ (written by the reference's
benchmarks/gen_torch_ref.py:61-173 with torch 2.9.1+rocm6.4, seed 42,
M=64, K=256, N=512; see meta.txt).  These are data files (inputs and
expected outputs), copied byte for byte; nothing of the reference is run.
MANIFEST.txt records the sha256 of every copied file.

Usage: python tests/golden/fetch_torch_ref.py [/path/to/reference]
"""
import hashlib
import os
import shutil
import sys

FILES = [
    "meta.txt",
    "x.bin",                 # X [64,256] bf16
    "w_gate.bin",            # W_gate [512,256] bf16
    "w_up.bin",              # W_up [512,256] bf16
    "w_down.bin",            # W_down [256,512] bf16
    "swiglu_bf16_trunc.bin", # S [64,512] bf16
    "h_gate_f32ref.bin",     # X.float() @ W_gate.float().T, f32 [64,512]
    "h_up_f32ref.bin",       # X.float() @ W_up.float().T, f32 [64,512]
    "h_gate_bf16acc.bin",    # torch.mm(X, W_gate.T) in bf16, stored f32
    "h_up_bf16acc.bin",      # torch.mm(X, W_up.T) in bf16, stored f32
    "y_bf16_f32acc.bin",     # S.float() @ W_down.float().T, f32 [64,256]
    "y_bf16chain.bin",       # torch.mm(S, W_down.T) in bf16, stored f32 [64,256]
]


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    src = os.path.join(ref, "benchmarks", "torch_ref")
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "torch_ref")
    os.makedirs(dst, exist_ok=True)
    lines = []
    for name in FILES:
        shutil.copyfile(os.path.join(src, name), os.path.join(dst, name))
        with open(os.path.join(dst, name), "rb") as f:
            digest = hashlib.sha256(f.read()).hexdigest()
        lines.append(f"{digest}  {name}")
    with open(os.path.join(dst, "MANIFEST.txt"), "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


if __name__ == "__main__":
    main()
