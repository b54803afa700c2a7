"""Merge-plan wire format, and replay of the TTT planner's trace records.

Two formats:

* **Plan files** (`save_plan` / `load_plan`): one safetensors file per plan.
  Every tensor field of a `TokenPlan` or `WeightedBilinearTokenPlan` is stored
  under its field name, bit for bit; the scalar fields, the names of the
  fields that are None and the plan's `metadata` travel as JSON in the
  file's header (key "vgo_plan").  `precomputed_qkv` and
  `source_attention_output` are activations of one forward, not part of a
  plan, and are not written.  A loaded plan drives the same kernels as the
  plan it was saved from and gives bit-identical compaction, attention and
  restore.
* **TTT trace records** (`read_ttt_trace`, `plan_from_ttt_record`,
  `load_ttt_trace`, `ttt_record_from_plan`, `save_ttt_trace`): the reference's
  `build_ttt_protected_uniform_convex_plan` appends one record per global
  layer (vggt_omega/models/sparse_convex.py:1907-1931) and saves
  `{"layers": records}` with torch.save (:77-80).  A record's source_ids,
  support_ids (patch-local ids), fp16 weights and accepted mask determine the
  plan the planner returns (:1932-1976); `plan_from_ttt_record` rebuilds it on
  the GPU with `vgo_sparse_convex_assemble` (keep, compact ids, parents,
  weights) and the deterministic mass kernel, so released TTT plans run on the
  same kernels as the planners built here.  Trace files are read with
  `torch.load(weights_only=True)`: nothing in them is executed.
"""
from __future__ import annotations

import dataclasses
import json
from pathlib import Path

import torch

from . import _lib
from .token_merging import TokenPlan, WeightedBilinearTokenPlan

FORMAT = "vgo-merge-plan"
VERSION = 1
_KINDS = {"TokenPlan": TokenPlan, "WeightedBilinearTokenPlan": WeightedBilinearTokenPlan}
_ACTIVATIONS = ("precomputed_qkv", "source_attention_output")

__all__ = ["save_plan", "load_plan", "read_ttt_trace", "plan_from_ttt_record", "load_ttt_trace",
           "ttt_record_from_plan", "save_ttt_trace"]


def _json_value(value):
    if isinstance(value, (bool, int, float, str)) or value is None:
        return value
    if isinstance(value, torch.Tensor) and value.numel() == 1:
        return value.item()
    if hasattr(value, "item"):  # numpy scalars
        return value.item()
    if isinstance(value, (list, tuple)):
        return [_json_value(v) for v in value]
    if isinstance(value, dict):
        return {str(k): _json_value(v) for k, v in value.items()}
    raise TypeError(f"plan metadata value {value!r} has no JSON form")


def save_plan(plan, path) -> None:
    """Write `plan` (TokenPlan or WeightedBilinearTokenPlan) to a safetensors file."""
    from safetensors.torch import save_file

    kind = type(plan).__name__
    if kind not in _KINDS:
        raise TypeError(f"save_plan takes a TokenPlan or WeightedBilinearTokenPlan, not {kind}")
    tensors, scalars, absent = {}, {}, []
    for f in dataclasses.fields(plan):
        if not f.init or f.name in _ACTIVATIONS or f.name == "metadata":
            continue
        value = getattr(plan, f.name)
        if value is None:
            absent.append(f.name)
        elif isinstance(value, torch.Tensor):
            # Own CPU copies: plans may share one tensor between fields.
            tensors[f.name] = value.detach().to("cpu", copy=True).contiguous()
        else:
            scalars[f.name] = _json_value(value)
    header = {"format": FORMAT, "version": VERSION, "kind": kind, "scalars": scalars,
              "absent": absent, "metadata": _json_value(dict(plan.metadata))}
    save_file(tensors, str(path), metadata={"vgo_plan": json.dumps(header, sort_keys=True)})


def load_plan(path, device=None):
    """Read a plan written by `save_plan`; tensors go to `device` (default: cuda:0)."""
    from safetensors import safe_open
    from safetensors.torch import load_file

    with safe_open(str(path), framework="pt") as handle:
        meta = handle.metadata() or {}
    if "vgo_plan" not in meta:
        raise ValueError(f"{path} is not a merge-plan file (no 'vgo_plan' header)")
    header = json.loads(meta["vgo_plan"])
    if header.get("format") != FORMAT or header.get("version") != VERSION:
        raise ValueError(f"unsupported merge-plan file: format {header.get('format')!r} "
                         f"version {header.get('version')!r}")
    cls = _KINDS.get(header.get("kind"))
    if cls is None:
        raise ValueError(f"unknown plan kind {header.get('kind')!r}")
    device = torch.device("cuda", 0) if device is None else torch.device(device)
    tensors = load_file(str(path), device=str(device))
    kwargs = dict(tensors)
    kwargs.update(header["scalars"])
    for name in header["absent"]:
        kwargs[name] = None
    kwargs["metadata"] = header["metadata"]
    names = {f.name for f in dataclasses.fields(cls) if f.init}
    unknown = set(kwargs) - names
    if unknown:
        raise ValueError(f"merge-plan file has fields {sorted(unknown)} unknown to {cls.__name__}")
    return cls(**kwargs)


# ------------------------------------------------------------ TTT traces ----
def read_ttt_trace(path) -> list[dict]:
    """The layer records of a trace file (reference sparse_convex.py:77-80)."""
    payload = torch.load(str(path), map_location="cpu", weights_only=True)
    if not isinstance(payload, dict) or not isinstance(payload.get("layers"), list):
        raise ValueError(f"{path} is not a TTT trace file (no 'layers' list)")
    return payload["layers"]


def _check_record(record: dict) -> tuple[int, int]:
    for key in ("frames", "patches", "source_ids", "support_ids", "weights", "accepted"):
        if key not in record:
            raise ValueError(f"TTT trace record has no '{key}'")
    frames, patches = int(record["frames"]), int(record["patches"])
    rows = record["source_ids"].numel()
    if (record["support_ids"].shape != (rows, 4) or record["weights"].shape != (rows, 4)
            or record["accepted"].shape != (rows,)):
        raise ValueError("TTT trace record needs source_ids [M], support_ids [M,4], weights [M,4], "
                         "accepted [M]")
    patch_count = frames * patches
    for key in ("source_ids", "support_ids"):
        ids = record[key]
        if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= patch_count):
            raise ValueError(f"TTT trace record {key} outside [0, {patch_count})")
    return frames, patches


@torch.no_grad()
def plan_from_ttt_record(record: dict, *, tokens_per_frame: int, patch_token_start: int,
                         device=None, preserve_queries: bool = False,
                         preserve_destination_keys: bool | None = None) -> WeightedBilinearTokenPlan:
    """The plan `build_ttt_protected_uniform_convex_plan` returned for this record.

    Reference sparse_convex.py:1932-1976: the accepted rows' sources leave the
    token set; keep = every other token in ascending order (special tokens and
    the remaining patches); parents = compact ids of the four supports, which
    must be kept ("protected TTT convex support must remain physical"); pool
    and restore weights = the record's weights; mass = the deterministic
    normalizer; key_log_mass = log(mass).
    """
    frames, patches = _check_record(record)
    if patch_token_start + patches != tokens_per_frame:
        raise ValueError("invalid protected TTT token layout")
    lib = _lib.load()
    device = torch.device("cuda", 0) if device is None else torch.device(device)
    if device.type != "cuda":
        raise RuntimeError("vgo kernels run on the GPU only; got a CPU device")
    total = frames * tokens_per_frame
    n = record["source_ids"].numel()

    def original(local: torch.Tensor) -> torch.Tensor:
        local = local.to(device=device, dtype=torch.int64)
        return (local // patches) * tokens_per_frame + patch_token_start + local % patches

    candidate = original(record["source_ids"])
    support = original(record["support_ids"]).contiguous()
    fit = record["accepted"].to(device=device, dtype=torch.float32)
    alpha = record["weights"].to(device=device, dtype=torch.float32).contiguous()
    keep_buf = torch.empty(total, device=device, dtype=torch.int64)
    o2c = torch.empty(total, device=device, dtype=torch.int64)
    source_buf = torch.empty(max(n, 1), device=device, dtype=torch.int64)
    parent_buf = torch.empty((max(n, 1), 4), device=device, dtype=torch.int64)
    weight_buf = torch.empty((max(n, 1), 4), device=device, dtype=torch.float32)
    stats = torch.zeros(4, device=device, dtype=torch.float32)
    stream = torch.cuda.current_stream(device).cuda_stream
    _lib.check(lib.vgo_sparse_convex_assemble(
        fit.data_ptr(), alpha.data_ptr(), support.data_ptr(), candidate.data_ptr(), None, 2.0,
        None, n, total, 0.5, keep_buf.data_ptr(), o2c.data_ptr(), source_buf.data_ptr(),
        parent_buf.data_ptr(), weight_buf.data_ptr(), stats.data_ptr(), stream))
    m = int(stats[0].item())
    parent = parent_buf[:m]
    if m and bool((parent < 0).any()):
        raise RuntimeError("protected TTT convex support must remain physical")
    weights = weight_buf[:m].view(1, m, 4)
    special = (torch.arange(frames, device=device)[:, None] * tokens_per_frame
               + torch.arange(patch_token_start, device=device)[None]).flatten()
    plan = WeightedBilinearTokenPlan(
        keep=keep_buf[:total - m].view(1, -1), source_original=source_buf[:m].view(1, -1),
        source_parent_compact=parent.view(1, m, 4), source_pool_weights=weights,
        source_restore_weights=weights, original_tokens=total,
        normalizer=torch.empty(0, device=device), preserve_queries=preserve_queries,
        preserve_destination_keys=(preserve_queries if preserve_destination_keys is None
                                   else preserve_destination_keys),
        dense_special_queries=True, special_query_original=special,
        special_query_compact=o2c.index_select(0, special),
        metadata={"planner": "ttt_trace_replay_v1", "layer": int(record.get("layer", 0)),
                  "merge_ratio": float(m / total)})
    mass, log_mass = plan.plan_mass()
    plan.normalizer = mass.view(1, -1, 1)
    plan.key_log_mass = log_mass.view(1, -1)
    return plan


def load_ttt_trace(path, *, tokens_per_frame: int, patch_token_start: int, device=None,
                   preserve_queries: bool = False) -> list[WeightedBilinearTokenPlan]:
    """One plan per layer record of a trace file."""
    return [plan_from_ttt_record(r, tokens_per_frame=tokens_per_frame,
                                 patch_token_start=patch_token_start, device=device,
                                 preserve_queries=preserve_queries)
            for r in read_ttt_trace(path)]


def ttt_record_from_plan(plan: WeightedBilinearTokenPlan, *, frames: int, tokens_per_frame: int,
                         patch_token_start: int, layer: int = 0) -> dict:
    """The trace fields a weighted plan determines (the inverse of plan_from_ttt_record).

    Sources and supports become patch-local ids, the weights fp16, every row
    accepted.  The planner's fit diagnostics (cosine, residual, bases) are not
    part of a plan and are not written.  A plan whose parents or sources
    include special tokens has no record form.
    """
    patches = tokens_per_frame - patch_token_start

    def local(ids: torch.Tensor) -> torch.Tensor:
        offset = ids % tokens_per_frame - patch_token_start
        if bool((offset < 0).any()):
            raise ValueError("special tokens have no patch-local id in a TTT trace record")
        return (ids // tokens_per_frame) * patches + offset

    parent = plan.source_parent_compact.reshape(-1, 4)
    if parent.numel() and bool((parent < 0).any()):
        raise ValueError("every source needs four parents in a TTT trace record")
    support = plan.keep.reshape(-1).index_select(0, parent.reshape(-1)).view(-1, 4)
    source = plan.source_original.reshape(-1)
    return {"layer": int(layer), "patches": patches, "frames": int(frames),
            "source_ids": local(source).to("cpu", torch.int32),
            "support_ids": local(support).to("cpu", torch.int32),
            "weights": plan.source_pool_weights.reshape(-1, 4).to("cpu", torch.float16),
            "accepted": torch.ones(source.numel(), dtype=torch.bool)}


def save_ttt_trace(records: list[dict], path) -> None:
    """Write records in the reference's trace-file layout (sparse_convex.py:77-80)."""
    torch.save({"layers": list(records)}, str(Path(path)))
