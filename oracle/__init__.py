"""CPU oracle of the quantized-linear path (TEST INFRASTRUCTURE ONLY).

A numpy restatement of the reference arithmetic used to check the HIP kernels.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only to check results or as the timed CPU
baseline; the ``vflash_amd`` package never imports it.

Modules:
  formats  -- bf16 / E4M3 / E2M1 rounding and decoding (OCP FP8 and MX specs)
  fp8      -- per-token quantization, W8A8 linear, epilogues (GELU-tanh,
              gate-residual, LoRA), merged QKV
  nvfp4    -- NVFP4 packing, 128x4 scale order, activation quantization, W4A8 and W4A4 linears
  baseline -- the reference's CPU weight-only dequant-matmul path (torch)
  fp8_torch -- fp8's rounding chains restated in torch for full-size checks on
              the device, pinned bit for bit against fp8 on the CPU

Pinning status of each function is stated in its docstring.
"""
