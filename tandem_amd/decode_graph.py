"""HIP-graph decode steps, one graph per batch-size bucket (python/tandem/executor/cuda_graph.py:1-154).

A decode step with b sequences replays the graph of the smallest bucket >= b (1, 2, 4, 8, 16, 24,
... up to max_bs). Graphs are captured from the largest bucket down into one shared memory pool,
after two eager warm-up passes on a side stream (the warm-up also allocates the split-K workspace
and sets up the kernels, which must not happen inside a capture). Per step, outside the graph, the
token ids are copied into the static input buffer (padding rows take token 0 and are computed but
never returned); then the bucket's graph replays and the first b rows of its output are returned.

Every W4Linear picks its kernel from the bucket's M at capture time, so each bucket replays the
kernels its table names for that batch size. The KV-cache plumbing of the reference runner (paged
layout, FlashInfer wrappers, the KV-split variants) belongs to the attention path, which this build
leaves out (see tandem_amd.model).
"""

from __future__ import annotations

import logging
from typing import Callable, Sequence

import torch
from torch import nn

logger = logging.getLogger(__name__)


def bucket_sizes(max_bs: int) -> list[int]:
    """1, 2, 4, 8, then every 8 from 16, ending at max_bs (python/tandem/executor/cuda_graph.py:34-38)."""
    if max_bs < 1:
        raise ValueError(f"max_bs must be >= 1 (got {max_bs})")
    sizes = [b for b in (1, 2, 4, 8) if b <= max_bs] + list(range(16, max_bs + 1, 8))
    if sizes[-1] != max_bs:
        sizes.append(max_bs)
    return sizes


class DecodeGraphRunner:
    """Bucketed HIP graphs of ``model(input_ids)`` (and ``model.compute_logits`` when ``logits``)."""

    def __init__(self, model: nn.Module, max_bs: int, device: torch.device, logits: bool = True) -> None:
        self.model = model
        self.device = device
        self.logits = logits
        self.sizes = bucket_sizes(max_bs)
        self.max_bs = self.sizes[-1]
        self.input_ids = torch.zeros(self.max_bs, dtype=torch.long, device=device)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.outputs: dict[int, torch.Tensor] = {}
        self._capture_all()

    def _fn(self, bs: int) -> Callable[[], torch.Tensor]:
        def run() -> torch.Tensor:
            hidden = self.model(self.input_ids[:bs])
            return self.model.compute_logits(hidden) if self.logits else hidden
        return run

    @torch.inference_mode()
    def _capture_all(self) -> None:
        pool = torch.cuda.graph_pool_handle()
        for bs in reversed(self.sizes):
            run = self._fn(bs)
            stream = torch.cuda.Stream(self.device)
            stream.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(stream):
                for _ in range(2):
                    run()
            torch.cuda.current_stream(self.device).wait_stream(stream)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=pool):
                self.outputs[bs] = run()
            self.graphs[bs] = graph
        torch.cuda.synchronize(self.device)
        logger.info("captured HIP graphs for decode batch sizes %s", self.sizes)

    def can_run(self, num_seqs: int) -> bool:
        return 1 <= num_seqs <= self.max_bs

    def bucket(self, num_seqs: int) -> int:
        return next(s for s in self.sizes if s >= num_seqs)

    @torch.inference_mode()
    def run(self, input_ids: Sequence[int] | torch.Tensor) -> torch.Tensor:
        """Token ids of b <= max_bs sequences -> the first b rows of the bucket's output (a view of a
        static buffer, overwritten by the next replay of that bucket)."""
        ids = torch.as_tensor(input_ids, dtype=torch.long)
        b = int(ids.numel())
        if not self.can_run(b):
            raise ValueError(f"decode batch {b} outside 1..{self.max_bs}")
        bs = self.bucket(b)
        padded = torch.zeros(bs, dtype=torch.long)
        padded[:b] = ids.reshape(-1).cpu()
        self.input_ids[:bs].copy_(padded.to(self.device, non_blocking=False))
        self.graphs[bs].replay()
        return self.outputs[bs][:b]
