"""Per-rank scenarios of the erasure-coded checkpoint manager, run in spawned
processes by test_checkpoint_cpu.py (gloo) and test_gpu_checkpoint.py."""
import os
import shutil
import sys
import traceback

import torch
import torch.distributed as dist

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def make_tensors(rank, device="cpu"):
    g = torch.Generator().manual_seed(100 + rank)
    sizes = [(3, 1000), (17,), (257, 33), (1,), (4096,), (5, 7, 11)]
    dts = [torch.float32, torch.bfloat16, torch.float32, torch.int64, torch.uint8, torch.float16]
    out = []
    for shp, dt in zip(sizes[: 3 + rank % 4], dts):
        x = torch.randn(shp, generator=g).to(dt) if dt.is_floating_point else \
            torch.randint(0, 200, shp, generator=g).to(dt)
        out.append(x.to(device))
    return out


def bump(t):
    """Change every element in place (an optimizer step)."""
    return t.add_(1) if t.is_floating_point() else t.bitwise_xor_(1)


def same(a, b):
    return len(a) == len(b) and all(
        x.dtype == y.dtype and x.shape == y.shape and
        torch.equal(x.cpu().reshape(-1).view(torch.uint8), y.cpu().reshape(-1).view(torch.uint8))
        for x, y in zip(a, b))


def lose_storage(mgr):
    """This rank's local checkpoint directory is gone (a replaced node)."""
    shutil.rmtree(mgr.local_dir)
    os.makedirs(mgr.local_dir)


class GroupSpy:
    """Reports the given process groups as NCCL (as the reference's
    data-parallel group is, megatron/core/parallel_state.py:730-736) and
    fails any CPU-tensor collective issued on them: the strategy must run
    its exchange on a gloo group of its own."""

    def __init__(self, groups):
        self.groups = [g for g in groups if g is not None]
        self.orig = {n: getattr(dist, n) for n in
                     ("get_backend", "all_gather", "all_reduce", "isend", "irecv", "barrier")}

    def __enter__(self):
        def backend(group=None):
            if any(group is g for g in self.groups):
                return "nccl"
            return self.orig["get_backend"](group)

        def guard(name):
            fn = self.orig[name]

            def wrapped(*a, **kw):
                g = kw.get("group")
                if any(g is x for x in self.groups):
                    raise AssertionError(f"dist.{name} on the NCCL coding group")
                return fn(*a, **kw)
            return wrapped

        dist.get_backend = backend
        for n in ("all_gather", "all_reduce", "isend", "irecv", "barrier"):
            setattr(dist, n, guard(n))
        return self

    def __exit__(self, *exc):
        for n, fn in self.orig.items():
            setattr(dist, n, fn)


def group_scenario(rank, world, root, scenario, unit, codec_cls, mods):
    """Coding groups other than the world: the reference's replication test
    runs cliques of ranks and loses ranks [6, 3, 4]
    (tests/unit_tests/dist_checkpointing/test_replication.py:75-80,146-160).

    strided  two data-parallel groups [0, 2, 4, 6] and [1, 3, 5, 7] (TP = 2),
             reported as NCCL: save, lose ranks 6, 3 and 4, load, concurrently
             in both groups, synchronously and staged in the background;
    cliques  the coding groups [2, 6, 7], [1, 3], [0, 4, 5] (uneven, not
             contiguous), each with its gloo twin passed as ``gloo_group``;
             lose ranks 6, 3 and 4, load."""
    CheckpointingException, ECLocalCheckpointManager, ErasureCodedStrategy, TensorListState = mods
    assert world == 8
    if scenario == "strided":
        layout = [[0, 2, 4, 6], [1, 3, 5, 7]]
    else:
        layout = [[2, 6, 7], [1, 3], [0, 4, 5]]
    # every rank creates every group, in the same order (as Megatron does)
    groups = [dist.new_group(g) for g in layout]
    twins = [dist.new_group(g, backend="gloo") for g in layout] if scenario == "cliques" else None
    gi = next(i for i, g in enumerate(layout) if rank in g)
    group, members = groups[gi], layout[gi]
    G = len(members)
    k, m = (2, 2) if G == 4 else (G - 1, 1)
    mine = make_tensors(rank)
    state = TensorListState([t.clone() for t in mine], {"rank": rank})
    spy = GroupSpy(groups if scenario == "strided" else [])
    with spy:
        if scenario == "strided":
            strat = ErasureCodedStrategy.from_ec_params(k, m, unit, jump=2, group=group,
                                                        codec=codec_cls(k, m, unit))
            assert strat.jump == 1, strat.jump          # global stride 2 = one member
            comm = strat.comm_group()
            assert comm is not group
            assert dist.get_process_group_ranks(comm) == members
        else:
            strat = ErasureCodedStrategy(k, m, unit, group=group, codec=codec_cls(k, m, unit),
                                         gloo_group=twins[gi])
            assert strat.comm_group() is twins[gi]
        mgr = ECLocalCheckpointManager(root, strat, stage_in_background=True)
        mgr.save(state, 1)
        idx = members.index(rank)
        names = sorted(f.name for f in mgr.local_dir.iterdir())
        want = sorted(f"iter_0000001_{members[(idx - p) % G]}_local.ec{p}" for p in range(k + m))
        assert names == want, (names, want)
        if scenario == "strided":
            # a background save in flight, then a foreground find_latest on the
            # same private group: the foreground waits for it
            req = mgr.save(state, 2, is_async=True)
            for t in state.tensors:
                bump(t)
            req.execute_sync()
            assert mgr.find_latest() == 2
        dist.barrier()   # world-wide, outside the spy's groups: every save is on disk
        if rank in (6, 3, 4):
            lose_storage(mgr)
        dist.barrier()
        it = mgr.find_latest()
        assert it == (2 if scenario == "strided" else 1), it
        got, name = mgr.load()
        assert name == f"iter_{it:07d}_{rank}_local", name
        assert same(got.tensors, mine) and got.common == {"rank": rank}
        if scenario == "strided":
            # a second manager over the same ranks shares the private group
            mgr2 = ECLocalCheckpointManager(root + "_b", ErasureCodedStrategy(
                k, m, unit, group=group, codec=codec_cls(k, m, unit)))
            mgr2.save(state, 7)
            got, _ = mgr2.load()
            assert same(got.tensors, state.tensors)


def run(rank, world, port, root, scenario, k, m, unit, use_gpu, errfile, jump=1):
    try:
        sys.path.insert(0, ROOT)
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        os.environ["MASTER_ADDR"] = "127.0.0.1"
        os.environ["MASTER_PORT"] = str(port)
        dist.init_process_group("gloo", rank=rank, world_size=world)
        import __graft_entry__
        __graft_entry__.load_package()
        from megatron_lm_amd.checkpoint import (CheckpointingException, ECLocalCheckpointManager,
                                                ErasureCodedStrategy, TensorListState)
        device = "cpu"
        if use_gpu:
            torch.cuda.set_device(0)
            device = "cuda:0"
            codec = None
            if scenario == "incremental":
                from megatron_lm_amd.checkpoint import GpuSliceCodec
                codec = GpuSliceCodec(k, m, unit, keep_block=True)
        else:
            from ec_cpu_codec import OracleSliceCodec
            codec = OracleSliceCodec(k, m, unit)
        if scenario in ("strided", "cliques"):
            from ec_cpu_codec import OracleSliceCodec
            group_scenario(rank, world, root, scenario, unit, OracleSliceCodec,
                           (CheckpointingException, ECLocalCheckpointManager,
                            ErasureCodedStrategy, TensorListState))
            dist.barrier()
            dist.destroy_process_group()
            return
        strat = ErasureCodedStrategy(k, m, unit, codec=codec, jump=jump)
        mgr = ECLocalCheckpointManager(root, strat,
                                       stage_in_background=scenario.startswith("background"))
        mine = make_tensors(rank, device)
        state = TensorListState([t.clone() for t in mine], {"rank": rank})

        if scenario == "recover":
            mgr.save(state, 1)
            dist.barrier()
            names = sorted(f.name for f in mgr.local_dir.iterdir())
            want = sorted(f"iter_0000001_{(rank - p * jump) % world}_local.ec{p}"
                          for p in range(k + m))
            assert names == want, (names, want)
            lost = [(world - 1) - 2 * i for i in range(m)]  # m ranks lose their storage
            if rank in lost:
                shutil.rmtree(mgr.local_dir)
                os.makedirs(mgr.local_dir)
            dist.barrier()
            assert mgr.find_latest() == 1
            got, name = mgr.load()
            assert name == f"iter_0000001_{rank}_local", name
            assert same(got.tensors, mine) and got.common == {"rank": rank}
        elif scenario == "loss_634":
            # The reference's loss pattern (test_replication.py:146-160): ranks
            # 6, 3 and 4 of 8 lose their local checkpoint; a code with m = 3
            # still loads iteration 1 on every rank.
            mgr.save(state, 1)
            dist.barrier()
            if rank in (6, 3, 4):
                lose_storage(mgr)
            dist.barrier()
            assert mgr.find_latest() == 1
            got, name = mgr.load()
            assert name == f"iter_0000001_{rank}_local" and same(got.tensors, mine)
        elif scenario in ("node_lost", "node_lost_adjacent"):
            # Two ranks per node, numbered node-major; node 1 (ranks 2, 3) loses
            # its storage.  With jump = 2 every rank's slices sit on distinct
            # nodes and the iteration loads; with jump = 1 a rank's slices
            # share a node and m = 1 cannot cover it.
            mgr.save(state, 1)
            dist.barrier()
            if rank in (2, 3):
                shutil.rmtree(mgr.local_dir)
                os.makedirs(mgr.local_dir)
            dist.barrier()
            if scenario == "node_lost":
                assert mgr.find_latest() == 1
                got, _ = mgr.load()
                assert same(got.tensors, mine)
            else:
                assert mgr.find_latest() == -1
        elif scenario == "tasd":
            # A tensor-aware state dict round trip: the object comes back with
            # its non-tensor part, the rebuilt tensors inserted, after a rank
            # lost its storage.
            from ec_tasd_double import FakeTensorAwareStateDict
            names = [f"t{i}" for i in range(len(mine))]
            common = {"rank": rank, "iteration": 5, "opt": {"lr": 1e-4, "betas": (0.9, 0.95)}}
            tasd = FakeTensorAwareStateDict([t.clone() for t in mine], common, names)
            kept = list(tasd.tensors)
            mgr.save(tasd, 5)
            assert not tasd.is_hollow and all(a is b for a, b in zip(tasd.tensors, kept))
            dist.barrier()
            if rank == world - 1:
                shutil.rmtree(mgr.local_dir)
                os.makedirs(mgr.local_dir)
            dist.barrier()
            got, name = mgr.load()
            assert isinstance(got, FakeTensorAwareStateDict), type(got)
            assert name == f"iter_0000005_{rank}_local" and not got.is_hollow
            assert got.common == common and got.names == names
            assert same(list(got.tensors), mine)
            sd = got.to_state_dict()
            assert sd["common"] == common and set(sd) == {"common", *names}
        elif scenario == "async_write_lost":
            # one rank's writer never ran: finalize fails on every rank and
            # leaves nothing of that iteration, the previous one stays
            mgr.save(state, 1)
            req = mgr.save(state, 2, is_async=True)
            if rank != 1:
                req.async_fn(*req.async_fn_args)
            dist.barrier()
            try:
                for fn in req.finalize_fns:
                    fn()
                raise AssertionError("finalize of an unwritten save did not raise")
            except CheckpointingException:
                pass
            names = {f.name for f in mgr.local_dir.iterdir()}
            assert not any(n.startswith("iter_0000002") for n in names), names
            assert mgr.find_latest() == 1
        elif scenario == "stray":
            # files of another group or another code in the directory are ignored
            mgr.save(state, 1)
            (mgr.local_dir / "iter_0000009_99_local.ec0").write_bytes(b"x" * 10)
            (mgr.local_dir / f"iter_0000009_{rank}_local.ec40").write_bytes(b"y" * 10)
            (mgr.local_dir / "notes.txt").write_bytes(b"z")
            dist.barrier()
            assert mgr.find_latest() == 1
            got, _ = mgr.load()
            assert same(got.tensors, mine)
        elif scenario == "cleanup":
            mgr.save(state, 1)
            mgr.save(state, 2)
            names = {f.name for f in mgr.local_dir.iterdir()}
            assert not any(n.startswith("iter_0000001") for n in names), names
            got, name = mgr.load()
            assert name.startswith("iter_0000002") and same(got.tensors, mine)
        elif scenario == "failed_save":
            mgr.save(state, 1)
            if rank == 1:
                strat.codec = type(strat.codec)(k, m, unit, fail=True)
            try:
                mgr.save(state, 2)
                raise AssertionError("save on a failing rank did not raise")
            except CheckpointingException:
                pass
            names = {f.name for f in mgr.local_dir.iterdir()}
            assert not any(n.startswith("iter_0000002") for n in names), names
            assert mgr.find_latest() == 1
        elif scenario == "too_many_lost":
            mgr.save(state, 1)
            dist.barrier()
            if rank < m + 1:
                shutil.rmtree(mgr.local_dir)
            dist.barrier()
            assert mgr.find_latest() == -1
            try:
                mgr.load()
                raise AssertionError("load with more than m losses did not raise")
            except CheckpointingException:
                pass
        elif scenario == "async":
            # What the reference's async queue does with the request
            # (megatron/core/dist_checkpointing/strategies/async_utils.py:498-519,
            # :172-206): add finalize functions, freeze, ship it without them
            # to a forked writer (or pickled to a spawned one), then finalize
            # on every rank.
            import pickle
            req = mgr.save(state, 3, is_async=True)
            assert len(req._fields) == 7 and req.async_fn is not None and req.preload_fn is None
            done = []
            req.add_finalize_fn(lambda: done.append(3))
            frozen = req.freeze()
            try:
                frozen.add_finalize_fn(lambda: None)
                raise AssertionError("a frozen request accepted a finalize function")
            except RuntimeError:
                pass
            ship = frozen._replace(call_idx=1, finalize_fns=[])
            pickle.dumps(ship)
            proc = torch.multiprocessing.get_context("fork").Process(
                target=ship.async_fn, args=ship.async_fn_args, kwargs=ship.async_fn_kwargs)
            proc.start()
            proc.join()
            assert proc.exitcode == 0
            dist.barrier()
            for fn in frozen.finalize_fns:
                fn()
            assert done == [3] and mgr.latest_iteration == 3
            got, name = mgr.load()
            assert name == f"iter_0000003_{rank}_local" and same(got.tensors, mine)
            # execute_sync: the same request run in place
            req = mgr.save(state, 4, is_async=True)
            req.execute_sync()
            names = {f.name for f in mgr.local_dir.iterdir()}
            assert not any(n.startswith("iter_0000003") for n in names), names
            got, name = mgr.load()
            assert name == f"iter_0000004_{rank}_local" and same(got.tensors, mine)
        elif scenario == "background":
            # A save staged in the background: save() returns once the state
            # is coded, the next optimizer step changes the tensors at once,
            # and the checkpoint still holds the state of the call.  The
            # request goes through the reference queue's steps (freeze, ship
            # without finalize functions to a writer, finalize on every rank).
            import pickle
            mgr.save(state, 1)
            req = mgr.save(state, 2, is_async=True)
            for t in state.tensors:
                bump(t)
            frozen = req.freeze()
            ship = frozen._replace(call_idx=1, finalize_fns=[])
            pickle.dumps(ship)
            if use_gpu:   # no fork of a process that holds the GPU
                ship.async_fn(*ship.async_fn_args, **ship.async_fn_kwargs)
            else:
                proc = torch.multiprocessing.get_context("fork").Process(
                    target=ship.async_fn, args=ship.async_fn_args, kwargs=ship.async_fn_kwargs)
                proc.start()
                proc.join()
                assert proc.exitcode == 0
            dist.barrier()
            for fn in frozen.finalize_fns:
                fn()
            assert mgr.latest_iteration == 2
            names = {f.name for f in mgr.local_dir.iterdir()}
            assert not any(n.startswith("iter_0000001") or n.startswith(".") for n in names), names
            got, name = mgr.load()
            assert name == f"iter_0000002_{rank}_local" and same(got.tensors, mine)
            # two saves in flight before either is finalized
            bumped = [t.clone() for t in state.tensors]
            r3 = mgr.save(state, 3, is_async=True)
            r4 = mgr.save(state, 4, is_async=True)
            r3.execute_sync()
            r4.execute_sync()
            assert mgr.latest_iteration == 4
            got, name = mgr.load()
            assert name == f"iter_0000004_{rank}_local" and same(got.tensors, bumped)
        elif scenario == "incremental":
            # Saves that name the tensors changed since the last save: the
            # first save is full, then one tensor changes per save, through
            # the synchronous, the async and the background path, and one
            # save changes nothing.  Every save loads back as the state of
            # its call, also after a rank loses its storage.  With the GPU
            # codec (keep_block) the later saves take the incremental path.
            delta = []
            if use_gpu:
                inner = strat.codec._snapshot_delta
                strat.codec._snapshot_delta = lambda *a, **kw: delta.append(1) or inner(*a, **kw)
            ts = state.tensors
            mgr.save(state, 1)
            bump(ts[0])
            mgr.save(state, 2, changed_tensors=[0])
            got, name = mgr.load()
            assert name == f"iter_0000002_{rank}_local" and same(got.tensors, ts)
            bump(ts[-1])
            mgr.save(state, 3, is_async=True, changed_tensors=[len(ts) - 1]).execute_sync()
            mgr.stage_in_background = True
            ts[1].view(-1)[:3] = 7   # part of a tensor
            mgr.save(state, 4, is_async=True, changed_tensors=[1]).execute_sync()
            mgr.save(state, 5, changed_tensors=[])
            if rank == world - 1:
                lose_storage(mgr)
            dist.barrier()
            got, name = mgr.load()
            assert name == f"iter_0000005_{rank}_local" and same(got.tensors, ts)
            if use_gpu:
                assert len(delta) == 4, delta
            else:
                assert strat.codec.changed_log == [None, [0], [len(ts) - 1], [1], []]
        elif scenario == "background_fail":
            # One rank fails before (fail) or during (fail_late) the
            # background staging: every rank's finalize raises, nothing of
            # that iteration is left, the previous one stays; then a good save.
            from ec_cpu_codec import OracleSliceCodec
            mgr.save(state, 1)
            for it, kw in ((2, {"fail": True}), (3, {"fail_late": True})):
                if rank == 1:
                    strat.codec = OracleSliceCodec(k, m, unit, **kw)
                req = mgr.save(state, it, is_async=True)
                try:
                    req.execute_sync()
                    raise AssertionError(f"background save with {kw} did not fail")
                except CheckpointingException:
                    pass
                names = {f.name for f in mgr.local_dir.iterdir()}
                assert not any(n.startswith(f"iter_{it:07d}") or n.startswith(".")
                               for n in names), names
                assert mgr.find_latest() == 1
                strat.codec = OracleSliceCodec(k, m, unit)
            mgr.save(state, 4, is_async=True).execute_sync()
            assert mgr.find_latest() == 4
        else:
            raise ValueError(scenario)
        dist.barrier()
        dist.destroy_process_group()
    except BaseException:
        with open(f"{errfile}.{rank}", "w") as f:
            f.write(traceback.format_exc())
        raise
