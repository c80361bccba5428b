"""testt_amd: MI355X (gfx950) kernels for the QLoRA fused-kernel set of SalReII/testt.

Drop-in for the kernel modules of the reference's `solution/` package (same module names,
functions, autograd.Function signatures and constants):

- nf4.py      NF4 double-quant unpack + frozen 4-bit linear (hipBLASLt GEMM)
- rmsnorm.py  residual add + RMSNorm, forward and backward
- rope.py     LoRA add + rotary + scatter of q/k/v to the attention's layout, fwd and bwd
- attention.py causal GQA flash attention (head dim 128), forward and backward
- mlp.py      gate/up GEMM + SwiGLU in fp16, gate/up kept (or recomputed) for backward
- head.py     fused head + loss + entropy + accuracy + per-row loss, no full logits
- warmup.py   start/wait hooks (the kernels are prebuilt, nothing compiles at run time)

The kernels are hand-written HIP in testt_amd/csrc, built into libsoupk.so behind the C ABI of
include/soupk.h (`python -m testt_amd.build_ext`) and called through ctypes with PyTorch's
current stream.  There is no CPU or Triton path.
"""

__all__ = ["apply", "configure_backward", "nf4", "rmsnorm", "rope", "attention", "mlp", "head",
           "warmup"]

# One process drives one GPU here, so autograd's per-device worker thread adds no parallelism,
# and handing every backward to it costs host time: on the MI355X boxes one decoder layer's
# eager forward + backward went from 823 to 682 us of wall time (host-bound to GPU-bound) with
# backward run on the calling thread.  apply() makes that the calling thread's setting.
SINGLE_THREADED_BACKWARD = True


def configure_backward(single_threaded=SINGLE_THREADED_BACKWARD):
    """Run autograd's backward passes started from this thread on this thread
    (torch.autograd.set_multithreading_enabled, a thread-local setting) instead of on the
    device's worker thread.  Results are the same either way."""
    import torch

    torch.autograd.set_multithreading_enabled(not single_threaded)


def apply():
    """Mirror of solution.apply() (solution/__init__.py:16-24).

    The reference installs four patches from its trainer_patch module (HF forward, TRL
    compute_loss, Soup rewind, Soup setup); that module and model.py stay the reference's own
    and import the kernel modules by name, so applying the reference's patches after placing
    these modules where solution/ keeps its kernels is the integration.  Here apply() loads the
    kernel library (loudly, if it is missing), runs the calling thread's backward passes on
    that thread (configure_backward) and then runs the trainer patches when a
    `trainer_patch` module sits beside this package, printing, as the reference does, any patch
    that cannot be installed."""
    from . import _ext

    _ext.lib()
    configure_backward()
    try:
        from . import trainer_patch  # noqa: F401  (present only in an integrated tree)
    except ImportError as exc:
        print(f"[testt_amd] trainer patches not installed: {exc!r}", flush=True)
        return
    for patch in (trainer_patch.patch_forward, trainer_patch.patch_sft_compute_loss,
                  trainer_patch.patch_rewind, trainer_patch.patch_setup):
        try:
            patch()
        except Exception as exc:  # noqa: BLE001 - a missing package must not stop `soup train`
            print(f"[testt_amd] {patch.__name__} not installed: {exc!r}", flush=True)
