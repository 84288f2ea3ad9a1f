"""One worker process of the shared-offload GPU test (run by tests/test_gpu_shared_offload.py).

Usage: shared_worker.py NAMESPACE PROFILE_DIR OUT_DIR WORKER_INDEX N_WORKERS LAYERS HIDDEN INTER SEED BUDGET

Builds a session, restores the model (creator: seeded weights; follower: a
meta skeleton), runs three streamed forwards, saves the outputs and its role,
then keeps its session open until every worker has saved its result.
"""

from __future__ import annotations

import os
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def main() -> int:
    ns, profile_dir, out_dir = sys.argv[1:4]
    index, n_workers, layers, hidden, inter, seed, budget = (int(v) for v in sys.argv[4:11])
    import torch

    from flextensor_amd import workloads as W
    from flextensor_amd.config import OffloadConfig
    from flextensor_amd.shared_offload import SharedOffloadSession

    print(f"worker {index}: start", flush=True)
    dev = torch.device("cuda", 0)
    cfg = OffloadConfig(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, max_gpu_mem_bytes=budget)

    def creator():
        return W.build_mlp_stack(layers, hidden, inter, seed=seed)

    def follower():
        with torch.device("meta"):
            return W.MLPStack(layers, hidden, inter)

    with SharedOffloadSession(ns, wait_timeout=120) as session:
        model = session.offload_from_profile(profile_dir, config=cfg, creator_model_factory=creator,
                                             follower_model_factory=follower)
        role = session.roles["default"]
        print(f"worker {index}: {role}", flush=True)
        x = W.mlp_input(16, hidden, seed=seed).to(dev)
        with torch.no_grad():
            outs = [model(x).cpu() for _ in range(3)]
        from flextensor_amd.manager import get_offload_manager

        mgr = get_offload_manager("default")
        info = {"role": role, "streamed": list(mgr.plan.streamed), "resident": list(mgr.plan.resident),
                "shm_blocks": sorted(getattr(mgr.controller, "shm_block_name_map", {}).values())}
        torch.save({"outs": outs, "info": info}, os.path.join(out_dir, f"w{index}.pt"))
        deadline = time.monotonic() + 120
        while sum(f.endswith(".pt") for f in os.listdir(out_dir)) < n_workers:
            if time.monotonic() > deadline:
                print(f"worker {index}: gave up waiting for the others", flush=True)
                return 3
            time.sleep(0.05)
    print(f"worker {index}: done", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
