"""Original-mode KV pool protocol (oracle), CPU.

Follows WanAttention in 投机采样/wam-p0-worktree/wan_va/modules/model.py:
  new_cache        :417-434   k, v [B, P, H, hd]; id [P] = -1; mask, is_pred False
  allocate_slots   :547-566   evict the `need` oldest ids when free < tokens
  next_cache_id    :568-575   max(valid id) + 1, or 0
  update_cache     :577-590   write K/V, mask True, id, is_pred = (update == 1)
  restore_cache    :592-593   mask False for the temporary slots
  clear_pred_cache :338-356   mask False where is_pred
The reference orders the eviction with torch.argsort, which is not stable: on
the CPU its order among equal ids is implementation-defined; on CUDA, at these
sizes, torch uses a stable radix sort (the reference's native path mirrors
that, 算子研究/wam_ops/baseline/csrc/block.cu:131-132).  order="stable" breaks
id ties by ascending slot (the CUDA behaviour, and the HIP kernel's);
order="torch" calls torch.argsort exactly as model.py:556-566 does.
"""
import torch


def new_cache(pool, heads, head_dim, batch=1, dtype=torch.float32):
    return {
        "k": torch.zeros(batch, pool, heads, head_dim, dtype=dtype),
        "v": torch.zeros(batch, pool, heads, head_dim, dtype=dtype),
        "id": torch.full((pool,), -1, dtype=torch.int64),
        "mask": torch.zeros(pool, dtype=torch.bool),
        "is_pred": torch.zeros(pool, dtype=torch.bool),
    }


def clone_cache(c):
    return {k: v.clone() for k, v in c.items()}


def allocate_slots(cache, tokens, order="stable"):
    mask, ids = cache["mask"], cache["id"]
    free = (~mask).nonzero().squeeze(-1)
    if free.numel() < tokens:
        used = mask.nonzero().squeeze(-1)
        if order == "torch":
            rank = torch.argsort(ids[used])
        else:  # (id, slot) ascending
            rank = torch.tensor(sorted(range(used.numel()), key=lambda i: (int(ids[used[i]]), int(used[i]))),
                                dtype=torch.long)
        need = tokens - free.numel()
        to_free = used[rank[:need]]
        mask[to_free] = False
        ids[to_free] = -1
        free = (~mask).nonzero().squeeze(-1)
    assert free.numel() >= tokens
    return free[:tokens]


def next_cache_id(cache):
    mask, ids = cache["mask"], cache["id"]
    return int(ids[mask].max()) + 1 if bool(mask.any()) else 0


def update_cache(cache, key, value, is_pred, order="stable"):
    """key/value [B, tokens, H, hd]; returns the slots written."""
    slots = allocate_slots(cache, key.shape[1], order)
    new_id = next_cache_id(cache)
    cache["k"][:, slots] = key.to(cache["k"].dtype)
    cache["v"][:, slots] = value.to(cache["v"].dtype)
    cache["mask"][slots] = True
    cache["id"][slots] = new_id
    cache["is_pred"][slots] = bool(is_pred)
    return slots


def restore_cache(cache, slots):
    cache["mask"][slots] = False


def clear_pred_cache(cache):
    cache["mask"][cache["is_pred"]] = False


def valid_slots(cache):
    return cache["mask"].nonzero().squeeze(-1)


def state_equal(a, b):
    """Pool state equality the reference's harness uses (tools/metrics.py:50-57):
    slots/id/mask/is_pred exactly and the K/V of valid slots."""
    if not (torch.equal(a["mask"], b["mask"]) and torch.equal(a["id"], b["id"])
            and torch.equal(a["is_pred"], b["is_pred"])):
        return False
    valid = valid_slots(a)
    return (torch.equal(a["k"][:, valid].float(), b["k"][:, valid].float())
            and torch.equal(a["v"][:, valid].float(), b["v"][:, valid].float()))
