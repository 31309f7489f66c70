"""BDDL task files: the problem, its regions, fixtures, objects and initial relations.

LIBERO describes each of its 130 tasks in a BDDL file (``libero/libero/bddl_files/<suite>/*.bddl``),
read by the reference through ``libero/libero/envs/bddl_utils.py`` (``robosuite_parse_problem``,
``get_regions:9-44``).  This reader produces the same content: regions keyed ``<target>_<region>``
with their ``ranges`` rectangles, ``yaw_rotation`` interval and ``rgba``; fixtures and objects by
category; the objects of interest; the initial relations (predicate names lower-cased) and the goal
expression.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
import re

_TOKEN = re.compile(r'\(|\)|[^\s()]+')


class BddlError(ValueError):
    pass


def parse_sexpr(text):
    """Nested lists of the parenthesised expression (comments after ';' dropped)."""
    text = '\n'.join(line.split(';', 1)[0] for line in text.splitlines())
    stack, top = [], []
    for tok in _TOKEN.findall(text):
        if tok == '(':
            stack.append(top)
            top = []
        elif tok == ')':
            if not stack:
                raise BddlError('unbalanced ")"')
            done, top = top, stack.pop()
            top.append(done)
        else:
            top.append(tok)
    if stack:
        raise BddlError('unbalanced "("')
    if len(top) != 1:
        raise BddlError('expected one top-level expression')
    return top[0]


def _number(tok):
    try:
        return float(tok)
    except ValueError:
        raise BddlError('not a number: %r' % tok)


@dataclass
class Region:
    name: str
    target: str
    ranges: list = field(default_factory=list)      # [(x0, y0, x1, y1)] in the target's frame
    yaw_rotation: tuple = (0.0, 0.0)
    rgba: tuple = (0.0, 0.0, 1.0, 0.0)


@dataclass
class Problem:
    name: str
    domain: str
    language: str
    regions: dict          # '<target>_<region>' -> Region
    fixtures: dict         # category -> [instance names]
    objects: dict          # category -> [instance names]
    obj_of_interest: list
    init: list             # (predicate, arg, ...) with the predicate lower-cased
    goal: list             # the goal expression as nested lists

    def category(self, instance):
        for table in (self.fixtures, self.objects):
            for cat, names in table.items():
                if instance in names:
                    return cat
        raise KeyError(instance)

    def is_fixture(self, instance):
        return any(instance in names for names in self.fixtures.values())


def _typed_list(items):
    """'a b - cat c - cat2' -> {cat: [a, b], cat2: [c]} (order kept)."""
    out, pending = {}, []
    it = iter(items)
    for tok in it:
        if tok == '-':
            cat = next(it, None)
            if cat is None or not pending:
                raise BddlError('dangling type marker')
            out.setdefault(cat, []).extend(pending)
            pending = []
        else:
            pending.append(tok)
    if pending:
        raise BddlError('untyped names %s' % pending)
    return out


def _regions(body):
    regions = {}
    for entry in body:
        if not isinstance(entry, list) or not entry:
            raise BddlError('bad region entry')
        name, target, ranges, yaw, rgba = entry[0], None, [], (0.0, 0.0), (0.0, 0.0, 1.0, 0.0)
        for attr in entry[1:]:
            key = attr[0]
            if key == ':target':
                target = attr[1]
            elif key == ':ranges':
                for rect in attr[1]:
                    if len(rect) != 4:
                        raise BddlError('a range is four numbers')
                    ranges.append(tuple(_number(x) for x in rect))
            elif key == ':yaw_rotation':
                vals = [_number(x) for x in attr[1][0]]
                yaw = (vals[0], vals[1])
            elif key == ':rgba':
                rgba = tuple(_number(x) for x in attr[1])
                if len(rgba) != 4:
                    raise BddlError('rgba is four numbers')
        if target is None:
            raise BddlError('region %s without a target' % name)
        regions[target + '_' + name] = Region(name, target, ranges, yaw, rgba)
    return regions


def _relation(expr):
    if not isinstance(expr, list) or not expr:
        raise BddlError('bad relation')
    return (expr[0].lower(),) + tuple(expr[1:])


def parse(source):
    """Parse a BDDL file (path) or text."""
    text = str(source)
    if '(define' not in text:
        text = Path(source).read_text()
    tree = parse_sexpr(text)
    if tree[0] != 'define':
        raise BddlError('expected (define ...)')
    name = domain = language = ''
    regions, fixtures, objects, interest, init, goal = {}, {}, {}, [], [], []
    for item in tree[1:]:
        head = item[0]
        if head == 'problem':
            name = item[1]
        elif head == ':domain':
            domain = item[1]
        elif head == ':language':
            language = ' '.join(str(x) for x in item[1:])
        elif head == ':regions':
            regions = _regions(item[1:])
        elif head == ':fixtures':
            fixtures = _typed_list(item[1:])
        elif head == ':objects':
            objects = _typed_list(item[1:])
        elif head == ':obj_of_interest':
            interest = list(item[1:])
        elif head == ':init':
            init = [_relation(e) for e in item[1:]]
        elif head == ':goal':
            goal = item[1] if len(item) > 1 else []
    if not name:
        raise BddlError('no problem name')
    return Problem(name, domain, language, regions, fixtures, objects, interest, init, goal)
