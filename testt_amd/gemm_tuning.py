"""hipBLASLt solution choices for the GEMMs of the QLoRA training step, replayed through PyTorch's
TunableOp (and by the layer's direct hipBLASLt calls, testt_amd/blas.py): hipBLASLt stays the
library, only the solution hipBLASLt's heuristic would pick is replaced by the one that timed
fastest for the problem on an MI355X.

hipBLASLt's first heuristic choice is far from its best solution on some of the step's shapes,
the worst being the gate|up input gradient ([2048 x 17920] @ [17920 x 1536]): 221 us with the
heuristic's 256x256 tile (48 tiles for 256 CUs) against about 150 us for its best listed
solution.

    enable()                      replay the committed table (tunableop_mi355x.csv here)
    python -m testt_amd.gemm_tuning --out PATH
                                  re-tune: one training step of the synthetic model with
                                  TunableOp tuning on, hipBLASLt solutions only

The table holds TunableOp's validators (torch, HIP, hipBLASLt versions, GPU arch); TunableOp
ignores a table whose validators do not match the running system, and problems not in the
table keep the heuristic's choice.  Any listed solution computes the same product, up to the
order of its fp32 sums.
"""

import argparse
import os
import sys

RESULTS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tunableop_mi355x.csv")


def enable(path=RESULTS):
    """Replay the tuned solutions of `path` for every torch.matmul of this process; True if
    TunableOp accepted the table."""
    import torch

    from . import blas

    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.tuning_enable(False)
    torch.cuda.tunable.record_untuned_enable(False)
    accepted = bool(torch.cuda.tunable.read_file(path))
    # the direct hipBLASLt GEMMs (testt_amd/blas.py) run the same solutions, once TunableOp
    # has checked the table's validators against this system
    if accepted:
        blas.load_table(path)
    else:
        blas.clear_table()
    return accepted


def disable():
    import torch

    from . import blas

    torch.cuda.tunable.enable(False)
    blas.clear_table()


def _write_table(path):
    import torch

    lines = [f"Validator,{k},{v}" for k, v in torch.cuda.tunable.get_validators()]
    lines += [",".join(str(x) for x in r) for r in torch.cuda.tunable.get_results()]
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def main(argv=None):
    ap = argparse.ArgumentParser(description="re-tune the training step's GEMMs (hipBLASLt)")
    ap.add_argument("--out", default=RESULTS)
    ap.add_argument("--layers", type=int, default=1,
                    help="decoder layers of the tuning model (they all share one set of shapes)")
    args = ap.parse_args(argv)
    # read by TunableOp when torch initialises it: hipBLASLt solutions only
    os.environ["PYTORCH_TUNABLEOP_ROCBLAS_ENABLED"] = "0"
    import torch

    from . import model, workloads

    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.tuning_enable(True)
    torch.cuda.tunable.set_filename(os.devnull)      # the table is written below, not at exit
    dev = torch.device("cuda", 0)
    hf = workloads.qwen2_qlora(dev, n_layers=args.layers)
    B, T = workloads.BATCH, workloads.SEQ
    g = workloads.gen(12)
    ids = torch.randint(0, workloads.VOCAB, (B, T), generator=g).to(dev)
    mask = torch.ones(B, T, dtype=torch.int64, device=dev)
    labels = ids.clone()
    labels[:, :T // 4] = -100
    for i in range(2):
        with torch.autocast("cuda", dtype=torch.float16):
            loss = model.fused_forward(hf, ids, mask, labels, None).loss
        loss.backward()
        torch.cuda.synchronize(dev)
        print(f"tuning step {i} done", flush=True)
    _write_table(args.out)
    print(f"wrote {len(torch.cuda.tunable.get_results())} problems to {args.out}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
