"""What sets the peak of one GPT-2-small training step, dense and compressed.

Builds the trainer's model (``train_gpt_lct.py``) with the caching
allocator's history recorded (``torch.cuda.memory._record_memory_history``),
runs two warm-up steps and one measured step, then replays the recorded
allocation and free events to find the moment in the measured step at which
the allocated total peaks.  The blocks live at that moment are grouped by the
innermost stack frame inside this repository, so the table says which tensors
the peak is made of: those held across steps (weights, optimizer state, the
TensorBuffer) and the step's own.

    python examples/nanogpt/memory_breakdown.py --mode both
"""
from __future__ import annotations

import argparse
import collections
import json
import sys
from pathlib import Path

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

import torch

from examples.nanogpt import train_gpt_lct as gpt

ROOT = Path(__file__).resolve().parents[2]
MIB = 2 ** 20


def _site(frames) -> str:
    """The innermost frame inside this repository, as file:line function."""
    for frame in frames:
        name = frame.get("filename", "")
        if name.startswith(str(ROOT)) and not name.endswith("memory_breakdown.py"):
            return f"{Path(name).relative_to(ROOT)}:{frame.get('line')} {frame.get('name')}"
    return "(no frame in this repository)"


PHASES = ("forward", "backward", "adam", "muon")


def _events(snapshot, device):
    """The allocation and free events of ``device`` in the recorded history."""
    return [ev for ev in snapshot["device_traces"][device.index]
            if ev["action"] in ("alloc", "free_requested")]


def _replay(events, bounds):
    """Replay every event.  ``bounds``: the event index at which each phase
    starts, and the index after the last.  Returns the total just before the
    first phase, each phase's peak total, and the live blocks {addr: (size,
    site)} at the highest of those peaks with its phase."""
    live: dict[int, tuple[int, str]] = {}
    total = 0
    held = 0
    peaks = [-1] * len(PHASES)
    best, at_best, best_phase = -1, {}, None
    for i, ev in enumerate(events):
        if i == bounds[0]:
            held = total
        if ev["action"] == "alloc":
            live[ev["addr"]] = (ev["size"], _site(ev.get("frames", [])))
            total += ev["size"]
        else:
            entry = live.pop(ev["addr"], None)
            if entry is not None:
                total -= entry[0]
        for k in range(len(PHASES)):
            if bounds[k] <= i < bounds[k + 1] and total > peaks[k]:
                peaks[k] = total
                if total > best:
                    best, at_best, best_phase = total, dict(live), PHASES[k]
    return held, peaks, at_best, best_phase


def measure(device, compressed: bool) -> dict:
    base = torch.cuda.memory_allocated(device)
    torch.cuda.memory._record_memory_history(max_entries=4_000_000)
    model, optimizers = gpt.build(device, compress_weights=compressed,
                                  compress_activations=compressed,
                                  compress_optimizer=compressed)
    for i in range(2):
        inputs, targets = gpt.random_tokens(gpt.BATCH, gpt.SEQ_LEN, device, seed=1000 + i)
        gpt.train_step(model, optimizers, inputs, targets)
    inputs, targets = gpt.random_tokens(gpt.BATCH, gpt.SEQ_LEN, device, seed=2000)
    torch.cuda.synchronize(device)
    # Where the measured step starts in the trace: a marker's address may also
    # belong to an earlier, freed allocation, so markers are searched after it.
    before = len(_events(torch.cuda.memory._snapshot(), device))
    # The measured step, phase by phase (train_gpt_lct.train_step's order);
    # a one-element allocation marks where each phase starts in the trace.
    markers = []

    def mark():
        markers.append(torch.empty(1, device=device))

    mark()
    loss = model(inputs, targets)
    mark()
    loss.backward()
    mark()
    optimizers[0].step()
    mark()
    optimizers[1].step()
    mark()
    model.zero_grad(set_to_none=True)
    torch.cuda.synchronize(device)
    snapshot = torch.cuda.memory._snapshot()
    torch.cuda.memory._record_memory_history(enabled=None)
    events = _events(snapshot, device)
    addresses = [m.data_ptr() for m in markers]
    bounds, k = [], 0
    for i in range(before, len(events)):
        ev = events[i]
        if k < len(addresses) and ev["action"] == "alloc" and ev["addr"] == addresses[k]:
            bounds.append(i + 1)
            k += 1
    if len(bounds) != len(addresses):
        raise RuntimeError("phase markers not found in the allocator trace")
    del markers
    held, peaks, at_peak, phase = _replay(events, bounds)
    by_site = collections.Counter()
    for size, site in at_peak.values():
        by_site[site] += size
    result = {
        "mode": "lct" if compressed else "dense",
        "allocated_before_build_mib": round(base / MIB, 1),
        "held_at_step_start_mib": round(held / MIB, 1),
        "phase_peaks_mib": {name: round(p / MIB, 1) for name, p in zip(PHASES, peaks)},
        "peak_phase": phase,
        "peak_by_site_mib": {site: round(size / MIB, 1)
                             for site, size in by_site.most_common() if size >= MIB // 2},
    }
    del model, optimizers
    torch.cuda.empty_cache()
    return result


def main():
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--mode", choices=("lct", "dense", "both"), default="both")
    args = parser.parse_args()
    if not torch.cuda.is_available():
        raise RuntimeError("needs a GPU")
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    for mode in (("dense", "lct") if args.mode == "both" else (args.mode,)):
        print(json.dumps(measure(device, mode == "lct"), indent=1), flush=True)


if __name__ == "__main__":
    main()
