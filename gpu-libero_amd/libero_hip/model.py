"""Model compiler: a :class:`~libero_hip.scene.Scene` -> flat MuJoCo-convention arrays.

This is the role of the reference's ``prepare``/``upload`` (``gpu/host/backends/cuda_fp32/model.py:27-219``)
and of the CPU MuJoCo compiler behind it.  It produces, in FP64:

* body / joint / dof / geom / site / actuator arrays in MuJoCo's meaning;
* the tree decomposition of the mass matrix (one dense block per kinematic tree) and the list of
  (dof, ancestor dof) pairs whose composite-rigid-body products fill those blocks;
* body levels (depth order) for level-parallel forward kinematics and DFS subtree sizes for subtree
  sums (bodies are in DFS preorder, so every subtree is a contiguous index range);
* the static collision pair table (contype/conaffinity, weld and parent filters), as the reference
  builds it at model time (``gpu/host/backends/cuda_fp32/model.py:171-191``);
* ``body_invweight0`` / ``dof_invweight0`` from M(qpos0), as MuJoCo's ``mj_setConst`` does;
* per-world capacities (``nconmax``, ``njmax``), cf. ``capacity_budget`` (``scene.py:71-86``).

Arrays are packed for the C ABI by :mod:`libero_hip.layout`.
"""
from __future__ import annotations

import math
import numpy as np

from . import scene as S


def quat2mat(q):
    w, x, y, z = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def qmul(a, b):
    return np.array(S._qmul(a, b))


def axis_angle_quat(axis, angle):
    s = math.sin(angle / 2)
    return np.array([math.cos(angle / 2), axis[0] * s, axis[1] * s, axis[2] * s])



def mesh_polygons(verts, tol=1e-9):
    """Faces of the convex hull of ``verts`` (the hull's own vertices) as polygons: coplanar hull
    triangles merged, each polygon's vertex indices counter-clockwise about its outward unit normal.
    Returns a list of (indices, normal)."""
    from scipy.spatial import ConvexHull
    v = np.asarray(verts, float)
    hull = ConvexHull(v)
    scale = float(np.abs(v).max()) or 1.0
    groups = []                               # (normal, offset, vertex set)
    for simplex, eq in zip(hull.simplices, hull.equations):
        n, off = eq[:3], eq[3]
        for g in groups:
            if np.dot(g[0], n) > 1.0 - tol and abs(g[1] - off) < tol * scale:
                g[2].update(int(i) for i in simplex)
                break
        else:
            groups.append([n / np.linalg.norm(n), off, set(int(i) for i in simplex)])
    out = []
    for n, off, ids in groups:
        ids = sorted(ids)
        centre = v[ids].mean(axis=0)
        u = v[ids[0]] - centre
        u /= np.linalg.norm(u)
        w = np.cross(n, u)
        ang = [np.arctan2(np.dot(v[i] - centre, w), np.dot(v[i] - centre, u)) for i in ids]
        order = [ids[k] for k in np.argsort(ang, kind='stable')]
        out.append((order, n))
    return out


def polygon_arrays(polys, vertnum):
    """Flatten per-mesh polygon lists into the model arrays: per mesh the polygon count and first
    polygon; per polygon its vertex list (mesh-local vertex indices), count and outward normal; per
    mesh vertex the polygons that contain it (mesh-local polygon ids, ascending)."""
    polynum, polyadr, vertadr, vertcnt, polyvert, normals = [], [], [], [], [], []
    mapadr, mapnum, polymap = [], [], []
    for mesh, (plist, nv) in enumerate(zip(polys, vertnum)):
        polyadr.append(len(vertcnt))
        polynum.append(len(plist))
        incident = [[] for _ in range(int(nv))]
        for pid, (ids, n) in enumerate(plist):
            vertadr.append(len(polyvert))
            vertcnt.append(len(ids))
            polyvert.extend(ids)
            normals.append(n)
            for i in ids:
                incident[i].append(pid)
        for lst in incident:
            mapadr.append(len(polymap))
            mapnum.append(len(lst))
            polymap.extend(lst)
    i32 = lambda x: np.array(x, np.int32)
    return dict(mesh_polynum=i32(polynum), mesh_polyadr=i32(polyadr), mesh_polyvertadr=i32(vertadr),
                mesh_polyvertnum=i32(vertcnt), mesh_polyvert=i32(polyvert),
                mesh_polynormal=np.array(normals, float).reshape(-1, 3), mesh_polymapadr=i32(mapadr),
                mesh_polymapnum=i32(mapnum), mesh_polymap=i32(polymap))


OSC_RANGE_KEYS = (('input_min', -1.0), ('input_max', 1.0),
                  ('output_min', [-0.05] * 3 + [-0.5] * 3), ('output_max', [0.05] * 3 + [0.5] * 3))


def osc_action_ranges(osc):
    """robosuite's Controller.scale_action ranges of the pose delta, as the reference packs them
    (osc_action_config, gpu/host/runtime/control/__init__.py:65-74): input_min, input_max,
    output_min, output_max, 6 values each (a scalar broadcasts), OSC_POSE's defaults for those the
    controller configuration omits.  Returns (scaled, ranges[24]): scaled is 1 when the
    configuration gives any range (the device then reads each world's osc_action_scale), else 0
    (the defaults, applied without reading the array).  Raises ValueError, as the reference, unless
    every value is finite and input_min < input_max."""
    values = [np.broadcast_to(np.asarray(osc.get(name, default), float), (6,)) for name, default in OSC_RANGE_KEYS]
    ranges = np.concatenate(values)
    if not np.isfinite(ranges).all() or np.any(values[0] >= values[1]):
        raise ValueError('OSC action ranges must be finite with input_min < input_max')
    return int(any(name in osc for name, _ in OSC_RANGE_KEYS)), ranges

class Model:
    """Compiled model: ``dims`` (ints), ``opt`` (scalars) and named numpy arrays."""

    def __init__(self, scene: S.Scene):
        self.scene = scene
        self.name = scene.name
        bodies = scene.bodies
        nbody = len(bodies)
        for b, body in enumerate(bodies[1:], start=1):
            if not 0 <= body.parent < b:
                raise ValueError('bodies must be in DFS preorder (parent before child)')
        parent = np.array([-1] + [bd.parent for bd in bodies[1:]], np.int32)
        # DFS preorder check: each subtree must be a contiguous index range
        subtree = np.ones(nbody, np.int32)
        for b in range(nbody - 1, 0, -1):
            subtree[parent[b]] += subtree[b]
        for b in range(1, nbody):
            p = parent[b]
            if not (p < b < p + subtree[p]):
                raise ValueError('bodies are not in DFS preorder')
        self.nbody = nbody
        a = {}
        a['body_parent'] = parent
        a['body_subtreesize'] = subtree
        root = np.zeros(nbody, np.int32)
        level = np.zeros(nbody, np.int32)
        for b in range(1, nbody):
            root[b] = b if parent[b] == 0 else root[parent[b]]
            level[b] = level[parent[b]] + 1
        a['body_rootid'] = root
        a['body_level'] = level
        a['body_pos'] = np.array([bd.pos for bd in bodies], float)
        a['body_quat'] = np.array([bd.quat for bd in bodies], float)
        a['body_ipos'] = np.array([bd.ipos for bd in bodies], float)
        a['body_iquat'] = np.array([bd.iquat for bd in bodies], float)
        a['body_mass'] = np.array([bd.mass for bd in bodies], float)
        a['body_inertia'] = np.array([bd.inertia for bd in bodies], float)
        smass = a['body_mass'].copy()
        for b in range(nbody - 1, 0, -1):
            smass[parent[b]] += smass[b]
        a['body_subtreemass'] = smass

        # joints and dofs
        jnt, jbody, jqadr, jdadr = [], [], [], []
        body_jntadr = np.full(nbody, -1, np.int32)
        body_jntnum = np.zeros(nbody, np.int32)
        body_dofadr = np.full(nbody, -1, np.int32)
        body_dofnum = np.zeros(nbody, np.int32)
        nq = nv = 0
        dof_body, dof_jnt = [], []
        for b, body in enumerate(bodies):
            if body.joints:
                body_jntadr[b] = len(jnt)
                body_dofadr[b] = nv
            for j in body.joints:
                if j.type == S.FREE and (parent[b] != 0 or len(body.joints) != 1):
                    raise ValueError('free joints must be the only joint of a child of the world')
                nqj, nvj = {S.FREE: (7, 6), S.BALL: (4, 3), S.SLIDE: (1, 1), S.HINGE: (1, 1)}[j.type]
                jnt.append(j)
                jbody.append(b)
                jqadr.append(nq)
                jdadr.append(nv)
                for _ in range(nvj):
                    dof_body.append(b)
                    dof_jnt.append(len(jnt) - 1)
                nq += nqj
                nv += nvj
            body_jntnum[b] = len(body.joints)
            body_dofnum[b] = nv - body_dofadr[b] if body.joints else 0
        self.nq, self.nv, self.njnt = nq, nv, len(jnt)
        a['body_jntadr'], a['body_jntnum'] = body_jntadr, body_jntnum
        a['body_dofadr'], a['body_dofnum'] = body_dofadr, body_dofnum
        a['jnt_type'] = np.array([j.type for j in jnt], np.int32)
        a['jnt_body'] = np.array(jbody, np.int32)
        a['jnt_qposadr'] = np.array(jqadr, np.int32)
        a['jnt_dofadr'] = np.array(jdadr, np.int32)
        a['jnt_limited'] = np.array([int(j.limited) for j in jnt], np.int32)
        a['jnt_pos'] = np.array([j.pos for j in jnt], float).reshape(-1, 3)
        a['jnt_axis'] = np.array([np.asarray(j.axis) / np.linalg.norm(j.axis) for j in jnt], float).reshape(-1, 3)
        a['jnt_range'] = np.array([j.range for j in jnt], float).reshape(-1, 2)
        a['jnt_stiffness'] = np.array([j.stiffness for j in jnt], float)
        a['jnt_margin'] = np.array([j.margin for j in jnt], float)
        a['jnt_solref'] = np.array([j.solref for j in jnt], float).reshape(-1, 2)
        a['jnt_solimp'] = np.array([j.solimp for j in jnt], float).reshape(-1, 5)
        qpos0 = np.zeros(nq)
        qpos_spring = np.zeros(nq)
        for k, j in enumerate(jnt):
            adr = jqadr[k]
            if j.type == S.FREE:
                qpos0[adr:adr + 3] = bodies[jbody[k]].pos
                qpos0[adr + 3:adr + 7] = bodies[jbody[k]].quat
                qpos_spring[adr:adr + 7] = qpos0[adr:adr + 7]
            elif j.type in (S.HINGE, S.SLIDE):
                qpos_spring[adr] = j.springref
        a['qpos0'], a['qpos_spring'] = qpos0, qpos_spring
        dof_body = np.array(dof_body, np.int32)
        dof_jnt = np.array(dof_jnt, np.int32)
        a['dof_body'], a['dof_jnt'] = dof_body, dof_jnt
        dof_parent = np.full(nv, -1, np.int32)
        last = np.full(nbody, -1, np.int32)          # last dof on the path world..body
        for b in range(1, nbody):
            prev = last[parent[b]]
            for d in range(body_dofadr[b], body_dofadr[b] + body_dofnum[b]):
                dof_parent[d] = prev
                prev = d
            last[b] = prev
        a['dof_parent'] = dof_parent
        a['body_lastdof'] = last
        chain = np.zeros(nbody, np.int32)
        for b in range(nbody):
            d = last[b]
            while d >= 0:
                chain[b] += 1
                d = dof_parent[d]
        self.maxchain = int(chain.max()) if nbody else 0
        a['dof_armature'] = np.array([jnt[dof_jnt[d]].armature for d in range(nv)], float)
        a['dof_damping'] = np.array([jnt[dof_jnt[d]].damping for d in range(nv)], float)
        a['dof_frictionloss'] = np.array([jnt[dof_jnt[d]].frictionloss for d in range(nv)], float)
        a['dof_solref'] = np.array([jnt[dof_jnt[d]].solref for d in range(nv)], float).reshape(-1, 2)
        a['dof_solimp'] = np.array([jnt[dof_jnt[d]].solimp for d in range(nv)], float).reshape(-1, 5)

        # trees: one dense mass block per child of the world that carries dofs
        tree_of_body = np.full(nbody, -1, np.int32)
        trees = []
        for b in range(1, nbody):
            if parent[b] == 0:
                dofs = [d for d in range(nv) if root[dof_body[d]] == b]
                if dofs:
                    if dofs != list(range(dofs[0], dofs[-1] + 1)):
                        raise ValueError('tree dofs must be contiguous')
                    trees.append((dofs[0], len(dofs)))
                    tree_of_body[b:b + subtree[b]] = len(trees) - 1
        self.ntree = len(trees)
        a['tree_dofadr'] = np.array([t[0] for t in trees], np.int32)
        a['tree_dofnum'] = np.array([t[1] for t in trees], np.int32)
        madr = np.zeros(len(trees), np.int32)
        for t in range(1, len(trees)):
            madr[t] = madr[t - 1] + trees[t - 1][1] ** 2
        a['tree_madr'] = madr
        self.nM = int(madr[-1] + trees[-1][1] ** 2) if trees else 0
        # trees with joint damping also get the block of M + h diag(damping) (implicit Euler), stored
        # after the mass blocks: its offset there, or -1
        dampadr, self.nMdamp = [], 0
        for adr, n in trees:
            if np.any(a['dof_damping'][adr:adr + n] > 0):
                dampadr.append(self.nMdamp)
                self.nMdamp += n * n
            else:
                dampadr.append(-1)
        a['tree_dampadr'] = np.array(dampadr, np.int32)
        self.maxtree = max((t[1] for t in trees), default=0)
        a['body_treeid'] = tree_of_body
        a['dof_treeid'] = tree_of_body[dof_body] if nv else np.zeros(0, np.int32)
        pairs_i, pairs_j = [], []
        for i in range(nv):
            j = i
            while j >= 0:
                pairs_i.append(i)
                pairs_j.append(j)
                j = dof_parent[j]
        a['mpair_i'] = np.array(pairs_i, np.int32)
        a['mpair_j'] = np.array(pairs_j, np.int32)
        self.nMpair = len(pairs_i)

        # level order for level-parallel kinematics
        nlevel = int(level.max()) if nbody > 1 else 0
        order = [b for lv in range(1, nlevel + 1) for b in range(1, nbody) if level[b] == lv]
        adr = [0]
        for lv in range(1, nlevel + 1):
            adr.append(adr[-1] + int(np.sum(level[1:] == lv)))
        a['level_adr'] = np.array(adr, np.int32)
        a['level_body'] = np.array(order, np.int32)
        self.nlevel = nlevel

        # geoms, sites, meshes
        geoms, gbody = [], []
        sites, sbody = [], []
        for b, body in enumerate(bodies):
            for g in body.geoms:
                geoms.append(g)
                gbody.append(b)
            for s in body.sites:
                sites.append(s)
                sbody.append(b)
        self.ngeom, self.nsite = len(geoms), len(sites)
        a['geom_type'] = np.array([g.type for g in geoms], np.int32)
        a['geom_body'] = np.array(gbody, np.int32)
        a['geom_contype'] = np.array([g.contype for g in geoms], np.int32)
        a['geom_conaffinity'] = np.array([g.conaffinity for g in geoms], np.int32)
        a['geom_condim'] = np.array([g.condim for g in geoms], np.int32)
        # frictionless (1) and sliding-friction (3) contacts: the kernels' row count per contact and
        # contact-space Jacobian (3 rows) assume condim <= 3
        bad = sorted(set(int(x) for x in a['geom_condim']) - {1, 3})
        if bad:
            raise ValueError('geom condim %s is not supported (1 or 3)' % bad)
        a['geom_priority'] = np.array([g.priority for g in geoms], np.int32)
        a['geom_pos'] = np.array([g.pos for g in geoms], float).reshape(-1, 3)
        a['geom_quat'] = np.array([g.quat for g in geoms], float).reshape(-1, 4)
        a['geom_size'] = np.array([g.size for g in geoms], float).reshape(-1, 3)
        a['geom_friction'] = np.array([g.friction for g in geoms], float).reshape(-1, 3)
        a['geom_solref'] = np.array([g.solref for g in geoms], float).reshape(-1, 2)
        a['geom_solimp'] = np.array([g.solimp for g in geoms], float).reshape(-1, 5)
        a['geom_solmix'] = np.array([g.solmix for g in geoms], float)
        a['geom_margin'] = np.array([g.margin for g in geoms], float)
        a['geom_gap'] = np.array([g.gap for g in geoms], float)
        meshes = []
        dataid = []
        for g in geoms:
            if g.type == S.MESH:
                dataid.append(len(meshes))
                meshes.append(np.asarray(g.vertices, float))
            else:
                dataid.append(-1)
        a['geom_dataid'] = np.array(dataid, np.int32)
        self.nmesh = len(meshes)
        a['mesh_vertnum'] = np.array([len(m) for m in meshes], np.int32)
        a['mesh_vertadr'] = np.concatenate([[0], np.cumsum(a['mesh_vertnum'])[:-1]]).astype(np.int32) \
            if meshes else np.zeros(0, np.int32)
        a['mesh_vert'] = np.concatenate(meshes).reshape(-1, 3) if meshes else np.zeros((0, 3))
        self.nmeshvert = len(a['mesh_vert'])
        # hull polygons (the faces the reference's plane_mesh manifold draws its contacts from)
        polys = [mesh_polygons(v) for v in meshes]
        a.update(polygon_arrays(polys, a['mesh_vertnum']))
        self.npoly = len(a['mesh_polyvertnum'])
        rbound, aabb = [], []
        for g, did in zip(geoms, dataid):
            if g.type == S.PLANE:
                rbound.append(0.0)
                aabb.append((0, 0, 0, 1e10, 1e10, 1e10))
            elif g.type == S.SPHERE:
                rbound.append(g.size[0])
                aabb.append((0, 0, 0) + (g.size[0],) * 3)
            elif g.type == S.CAPSULE:
                rbound.append(g.size[0] + g.size[1])
                aabb.append((0, 0, 0, g.size[0], g.size[0], g.size[0] + g.size[1]))
            elif g.type == S.BOX:
                rbound.append(float(np.linalg.norm(g.size)))
                aabb.append((0, 0, 0) + tuple(g.size))
            elif g.type == S.MESH:
                v = meshes[did]
                rbound.append(float(np.linalg.norm(v, axis=1).max()))
                lo, hi = v.min(axis=0), v.max(axis=0)
                aabb.append(tuple((lo + hi) / 2) + tuple((hi - lo) / 2))
            else:
                raise ValueError('unsupported geom type %d' % g.type)
        a['geom_rbound'] = np.array(rbound, float)
        a['geom_aabb'] = np.array(aabb, float).reshape(-1, 6)
        a['site_body'] = np.array(sbody, np.int32)
        a['site_pos'] = np.array([s.pos for s in sites], float).reshape(-1, 3)
        a['site_quat'] = np.array([s.quat for s in sites], float).reshape(-1, 4)

        # actuators (joint transmission; motor or position servo)
        acts = scene.actuators
        self.nu = len(acts)
        a['actuator_trnid'] = np.array([ac.joint for ac in acts], np.int32)
        a['actuator_gear'] = np.array([ac.gear for ac in acts], float)
        a['actuator_gainprm'] = np.array([1.0 if ac.kind == 'motor' else ac.kp for ac in acts], float)
        a['actuator_biasprm'] = np.array([(0.0, 0.0, 0.0) if ac.kind == 'motor' else (0.0, -ac.kp, -ac.kv)
                                          for ac in acts], float).reshape(-1, 3)
        a['actuator_biastype'] = np.array([0 if ac.kind == 'motor' else 1 for ac in acts], np.int32)
        a['actuator_ctrlrange'] = np.array([ac.ctrlrange for ac in acts], float).reshape(-1, 2)
        a['actuator_forcerange'] = np.array([ac.forcerange for ac in acts], float).reshape(-1, 2)
        a['actuator_ctrllimited'] = np.ones(self.nu, np.int32)
        a['actuator_forcelimited'] = np.array([int(ac.forcelimited) for ac in acts], np.int32)

        # gravity compensation (MuJoCo body_gravcomp, jnt_actgravcomp)
        a['body_gravcomp'] = np.array([bd.gravcomp for bd in bodies], float)
        a['jnt_actgravcomp'] = np.array([int(j.actuatorgravcomp) for j in jnt], np.int32)
        self.has_gravcomp = int(bool(np.any(a['body_gravcomp'][1:] != 0)))
        # inertia-box fluid forces (MuJoCo mj_passive): on when the medium has density or viscosity
        self.has_fluid = int(scene.options.density > 0 or scene.options.viscosity > 0)
        # force / torque sensors at sites, three values each
        sens = list(getattr(scene, 'sensors', []) or [])
        kinds = {'force': 4, 'torque': 5}
        for s in sens:
            if s.kind not in kinds or not 0 <= s.site < self.nsite:
                raise ValueError('sensors are force or torque sensors at a site')
        self.nsensor = len(sens)
        self.nsensordata = 3 * len(sens)
        a['sensor_type'] = np.array([kinds[s.kind] for s in sens], np.int32)
        a['sensor_objid'] = np.array([s.site for s in sens], np.int32)
        a['sensor_adr'] = np.array([3 * k for k in range(len(sens))], np.int32)
        a['sensor_datatype'] = np.zeros(len(sens), np.int32)
        a['sensor_cutoff'] = np.array([s.cutoff for s in sens], float)

        # OSC configuration (one robot: n arm dofs, the eef site, n arm + 2 gripper actuators)
        osc = scene.osc
        arm = osc['arm_joints']
        self.osc_ndof = len(arm)
        if not 1 <= self.osc_ndof <= 8 or len(osc['actuators']) != self.osc_ndof + 2:
            raise ValueError('the controller drives 1 to 8 arm joints and two gripper actuators')
        a['osc_qposadr'] = np.array([jqadr[j] for j in arm], np.int32)
        a['osc_dofadr'] = np.array([jdadr[j] for j in arm], np.int32)
        a['osc_actuator'] = np.array(osc['actuators'], np.int32)
        self.osc_site = int(osc['site'])
        self.osc_uncouple = int(osc.get('uncouple', 1))
        self.osc_gripper_speed = float(osc.get('gripper_speed', 0.01))
        self.osc_action_scaled, self.osc_action_scale = osc_action_ranges(osc)

        self.arrays = a
        self.opt = scene.options
        weld = np.zeros(nbody, np.int32)
        for b in range(1, nbody):
            weld[b] = b if body_jntnum[b] else weld[parent[b]]
        a['body_weldid'] = weld
        self._pairs()
        self._invweight0()
        opts = self.opt
        self.nconmax = int(opts.nconmax)
        dim = int(a['geom_condim'].max()) if self.ngeom else 1
        rows_per_contact = dim if opts.cone == S.ELLIPTIC else max(1, 2 * (dim - 1))
        self.rows_per_contact = rows_per_contact
        if opts.disableflags & S.DISABLE_CONSTRAINT:
            self.njmax = 0
        else:
            self.njmax = int(opts.njmax) if opts.njmax else rows_per_contact * self.nconmax + 2 * nv
        # per-world activity (heterogeneous batches): bodies of inactive objects are frozen
        self.body_active = scene.body_active

    def _pairs(self):
        """Static candidate pair table: MuJoCo's contype/conaffinity, weld and parent filters."""
        a = self.arrays
        g1s, g2s = [], []
        parent, weld = a['body_parent'], a['body_weldid']
        for g1 in range(self.ngeom):
            for g2 in range(g1 + 1, self.ngeom):
                b1, b2 = a['geom_body'][g1], a['geom_body'][g2]
                w1, w2 = weld[b1], weld[b2]
                if w1 == w2:
                    continue                       # same rigid body (incl. both static)
                if not ((a['geom_contype'][g1] & a['geom_conaffinity'][g2]) or
                        (a['geom_contype'][g2] & a['geom_conaffinity'][g1])):
                    continue
                pw1, pw2 = weld[parent[w1]] if w1 else 0, weld[parent[w2]] if w2 else 0
                if (w1 != 0 and pw2 == w1 and w2 != 0) or (w2 != 0 and pw1 == w2 and w1 != 0):
                    continue                       # parent-child filter (not for the world)
                t1, t2 = a['geom_type'][g1], a['geom_type'][g2]
                if t1 > t2:                          # canonical order: lower type first
                    g1s.append(g2)
                    g2s.append(g1)
                else:
                    g1s.append(g1)
                    g2s.append(g2)
        a['pair_geom'] = np.array(list(zip(g1s, g2s)), np.int32).reshape(-1, 2)
        self.npair = len(g1s)
        # largest union of the two bodies' dof chains over the pair table (contact Jacobian width)
        def chain(b):
            out, d = [], a['body_lastdof'][b]
            while d >= 0:
                out.append(int(d))
                d = a['dof_parent'][d]
            return set(out)
        widths = [len(chain(a['geom_body'][x]) | chain(a['geom_body'][y])) for x, y in zip(g1s, g2s)]
        self.maxpairdof = max(widths, default=1) or 1
        # Box-box goes through GJK/EPA and the box manifold unless a box has a margin or native CCD
        # is disabled (gpu/host/backends/cuda_fp32/physics.py:90); EPA runs 16 iterations when every
        # convex pair is box-box, else ccd_iterations (gpu/host/runtime/collision/mjwarp_convex_collision.py:79).
        gt = a['geom_type']
        has_boxbox_margin = any(gt[g] == S.BOX and a['geom_margin'][g] > 0 for g in range(self.ngeom))
        # MuJoCo 2.3.7 semantics (opt.mpr): convex pairs by MPR, box-box always by the primitive routine
        self.convex_mpr = int(bool(getattr(self.opt, 'mpr', False)))
        self.boxbox_primitive = int(has_boxbox_margin or bool(self.opt.disableflags & S.DISABLE_NATIVECCD)
                                    or self.convex_mpr)
        convex = [(gt[x], gt[y]) for x, y in zip(g1s, g2s)
                  if (gt[x], gt[y]) != (S.BOX, S.BOX) or not self.boxbox_primitive]
        convex = [t for t in convex if t[0] != S.PLANE and (S.MESH in t or t == (S.BOX, S.BOX))]
        all_box = bool(convex) and all(t == (S.BOX, S.BOX) for t in convex)
        self.epa_iterations = 16 if all_box else int(self.opt.ccd_iterations)

    def _invweight0(self):
        """body_invweight0 and dof_invweight0 from J M(qpos0)^-1 J^T, as in mj_setConst."""
        from .kinematics_host import forward_host
        a = self.arrays
        fk = forward_host(self, self.arrays['qpos0'])
        M = fk['M_dense']
        nv = self.nv
        Minv = np.linalg.inv(M) if nv else np.zeros((0, 0))
        biw = np.zeros((self.nbody, 2))
        for b in range(1, self.nbody):
            jacp, jacr = fk['jac'](b, fk['xipos'][b])
            J = np.vstack([jacp, jacr])
            if not np.any(J):
                continue
            A = J @ Minv @ J.T
            biw[b] = (np.trace(A[:3, :3]) / 3, np.trace(A[3:, 3:]) / 3)
        a['body_invweight0'] = biw
        diw = np.zeros(nv)
        for j in range(self.njnt):
            d = a['jnt_dofadr'][j]
            if a['jnt_type'][j] == S.FREE:
                diw[d:d + 3] = np.mean(np.diag(Minv)[d:d + 3])
                diw[d + 3:d + 6] = np.mean(np.diag(Minv)[d + 3:d + 6])
            else:
                diw[d] = Minv[d, d]
        a['dof_invweight0'] = diw
        # mean diagonal inertia at qpos0 (MuJoCo stat.meaninertia), the Newton solver's scale
        self.meaninertia = float(np.mean(np.diag(M))) if nv else 1.0

    # ---------------------------------------------------------------- convenience
    def initial_state(self):
        """(nworld, 1+nq+nv) LIBERO flat states [time | qpos | qvel]."""
        sc = self.scene
        return np.concatenate([np.zeros((sc.nworld, 1)), sc.init_qpos, sc.init_qvel], axis=1)

    def summary(self):
        return dict(name=self.name, nq=self.nq, nv=self.nv, nu=self.nu, nbody=self.nbody,
                    ngeom=self.ngeom, nsite=self.nsite, npair=self.npair, nM=self.nM,
                    ntree=self.ntree, nconmax=self.nconmax, njmax=self.njmax)
