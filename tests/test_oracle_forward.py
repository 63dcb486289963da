"""The oracle's two forward passes agree: the paged path over this engine's
packs (borrowed prefix pages, scatter maps, block tables) and each
document's prompt run whole. Runs on the CPU with the tiny configuration,
so pack metadata is pinned numerically without a GPU."""

import torch

from oracle import qwen3_ref as ref
from quail_amd.arena import KVArena
from quail_amd.chunk import pack_chunk
from quail_amd.model import CONFIGS, build_synthetic
from quail_amd.prefix import PrefixIndex
from quail_amd.workload import make_workload
from tests.helpers import admit, pack_specs, ref_model


def test_paged_pack_forward_equals_whole_documents():
    cfg = CONFIGS["tiny"]
    wl = make_workload("tiny", seed=3, documents=10)
    model = build_synthetic(cfg, seed=3, device="cpu", norm_init="random")
    m = ref_model(model)
    arena = KVArena(cfg.layers, 96, 16, cfg.kv_heads, cfg.head_dim, device="cpu")
    prefixes, suffixes = wl.groups_input()
    tree = PrefixIndex(wl.prompts).tree(16)
    # a small budget forces several packs; children borrow pages written by
    # an earlier pack
    adm = admit(prefixes, suffixes, arena, 400, tree=tree)
    pools = [(torch.zeros(96 * 16, cfg.kv_heads, cfg.head_dim, dtype=torch.bfloat16),
              torch.zeros(96 * 16, cfg.kv_heads, cfg.head_dim, dtype=torch.bfloat16))
             for _ in range(cfg.layers)]
    got = {}
    packs = 0
    while not adm.done():
        groups = adm.next_chunk(arena.free_pages)
        assert groups and not adm.take_prefills()
        chunk = pack_chunk(arena, pack_specs(adm, groups))
        normed = ref.forward_chunk(m, chunk.host_ids, chunk.host_positions,
                                   chunk.final_indices, chunk.meta["unified"], pools, 16)
        for i, (d, first, end, _) in enumerate(groups):
            got[d] = normed[i]
            adm.report(d, first, end, [True])
        packs += 1
    assert packs >= 2
    assert adm.borrowed_tokens > 0
    dense = ref.forward_documents(m, wl.prompts)
    paged = torch.stack([got[d] for d in range(len(wl.prompts))])
    torch.testing.assert_close(paged.float(), dense.float(), rtol=0.02, atol=0.02)
    rows = m.head[[10, 11]]
    y1, n1, _, _ = ref.answer(paged, rows, [1, 0])
    y2, n2, _, _ = ref.answer(dense, rows, [1, 0])
    assert ((y1 - n1) - (y2 - n2)).abs().max().item() <= 0.05
