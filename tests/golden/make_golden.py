"""Write the golden fixtures of this directory from torch's CPU routines.

  gelu_tanh_bf16.npy  uint16[65536]: torch.nn.functional.gelu(x, approximate="tanh") for every
                      bfloat16 bit pattern x, one vectorised CPU call. The reference applies this
                      routine to bfloat16 activations (backends/turbo/vendor/comfy_kitchen/
                      backends/_activations.py:47-48).
  silu_bf16.npy       uint16[65536]: torch.nn.functional.silu(x) for every bfloat16 bit pattern x,
                      the gate activation of the reference's SwiGLU (backends/turbo/vendor/
                      comfy_kitchen/backends/_activations.py:50-52).
  e4m3fn_to_f32.npy   float32[256]: torch's float8_e4m3fn -> float32 conversion of every code, as
                      the reference's decode uses for fp8 group scales (backends/turbo/vendor/
                      comfy_kitchen/backends/eager/w4a8_int8.py:361).

Run: python tests/golden/make_golden.py
"""

import pathlib

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent


def main() -> None:
    bits = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16)
    y = torch.nn.functional.gelu(bits.view(torch.bfloat16), approximate="tanh")
    np.save(HERE / "gelu_tanh_bf16.npy", y.view(torch.int16).numpy().view(np.uint16))
    y = torch.nn.functional.silu(bits.view(torch.bfloat16))
    np.save(HERE / "silu_bf16.npy", y.view(torch.int16).numpy().view(np.uint16))
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    np.save(HERE / "e4m3fn_to_f32.npy", codes.view(torch.float8_e4m3fn).float().numpy())
    print("wrote", sorted(p.name for p in HERE.glob("*.npy")))


if __name__ == "__main__":
    main()
